"""The C-ABI library loads on a machine without a GPU and exports every entry
point include/gsample.h declares (no compute calls here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gsample.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|double|float|void\s*\*|const char\s*\*)\s+(gs_\w+)\s*\(", text, re.M)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for required in ("gs_create", "gs_sample", "gs_build_masks", "gs_lmhead", "gs_token_log_prob"):
        assert required in names


@pytest.mark.parametrize("name", ["libgsample.so", "libgsample_checked.so"])
def test_library_exports_every_declared_symbol(name):
    """The library and its checked build (range-checked finish indices)."""
    import gsample.runtime as rt

    path = os.path.join(os.path.dirname(rt.LIB_PATH), name)
    if not os.path.exists(path):
        pytest.fail(f"{name} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) <= set(rt.EXPORTED_SYMBOLS) | set(declared_functions())


def test_host_math_exports_match_the_oracle(oracle):
    """The library's host-callable js_exp/js_log/SeededRandom/softcap (the code the
    kernels compile) agree with the oracle bit for bit; needs no GPU."""
    import numpy as np

    import gsample.runtime as rt

    lib = rt.library()
    rng = np.random.default_rng(7)
    xs = np.concatenate([rng.normal(0, 20, 20000), -np.abs(rng.normal(0, 300, 2000)), [0.0, -0.0, 1e-300, 700.0]])
    for x in xs:
        assert np.float64(lib.gs_js_exp(x)).view(np.uint64) == np.float64(oracle.js_exp(x)).view(np.uint64)
        if x > 0:
            assert np.float64(lib.gs_js_log(x)).view(np.uint64) == np.float64(oracle.js_log(x)).view(np.uint64)
    for seed in (0, 42, -9, 2 ** 35):
        for i in (0, 1, 2, 1000, 4_000_000):
            assert lib.gs_seeded_random(seed, i) == oracle.draw(seed, i)
    # the final-logit softcap: bit for bit with the oracle's, over the normal,
    # tiny (series branch), saturated and special inputs
    xs32 = np.concatenate([rng.normal(0, 25, 20000), rng.normal(0, 1e-3, 2000), [0.0, -0.0, 1e-30, 3000.0, -3000.0,
                                                                                  np.inf, -np.inf]]).astype(np.float32)
    for cap in (30.0, 50.0, 7.5):
        ref = oracle.softcap(xs32, cap)
        got = np.array([lib.gs_softcap(float(x), cap) for x in xs32], dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), cap


def test_config_validation_messages_through_the_abi():
    """gs_validate_configs returns the reference's joined message
    (decoding.ts:34-57, generation-config.ts:65); host-only, no GPU."""
    import ctypes as C

    import numpy as np

    import gsample.runtime as rt

    lib = rt.library()
    cfg = np.zeros(1, dtype=rt.ROW_CONFIG_DTYPE)
    cfg["temperature"] = 0.5
    cfg["top_p"] = np.nan
    cfg["repetition_penalty"] = 1.0
    cfg["typical_p"] = 1.0
    cfg["repetition_window"] = -1
    cfg["frequency_penalty"] = np.inf
    cfg["presence_penalty"] = -0.1
    st = lib.gs_validate_configs(None, C.c_void_p(cfg.ctypes.data), 1)
    assert st == 2
    assert lib.gs_last_error(None).decode() == (
        "Invalid Gemma decoding config: topP must be between 0 and 1; repetitionWindow must be a non-negative "
        "integer; frequencyPenalty must be finite and non-negative; presencePenalty must be finite and non-negative")
