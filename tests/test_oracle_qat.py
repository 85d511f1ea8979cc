"""The int2 QAT linear oracle (oracle/qat_ref.c, restating
src/reference/qat-linear.ts:45-148) against the reference's own known
answers: tests/qat-linear.spec.ts:20-90 (packing order, the int2 midpoint
zero point with a row scale, SRQ ties-to-even and clamping, the shape and
code errors) and the int2 LM-head GPU test's expected logits
(tests/qat-linear-gpu.spec.ts:1307-1397: rows of codes 2 / 3 / 1 over an
all-ones activation give 0 / 768 / -384)."""
import numpy as np
import pytest

from oracle import oracle


def test_packs_int2_low_to_high_bits():
    codes = [0, 1, 2, 3, 3, 2, 1, 0, 1, 3, 0, 2, 2, 0, 3, 1]
    packed = oracle.pack_int2_rows(codes, 1, 16)
    assert packed.tolist() == [0x728D1BE4]
    assert all(oracle.unpack_int2(packed, i) == c for i, c in enumerate(codes))


def test_int2_midpoint_zero_point_and_row_scale():
    x = np.array([1, -2, 3, -4, 5, -6, 7, -8, 9, -10, 11, -12, 13, -14, 15, -16], np.float32)
    codes = [0, 1, 2, 3, 3, 2, 1, 0, 1, 3, 0, 2, 2, 0, 3, 1]
    explicit = sum((c - 2) * float(v) for c, v in zip(codes, x))
    out = oracle.qat_linear_int2(x, oracle.pack_int2_rows(codes, 1, 16), [0.25], 16, 1)
    assert out.tolist() == [np.float32(explicit * 0.25)]


def test_srq_ties_to_even_and_clamp():
    assert oracle.apply_srq(2.5, 1) == 2
    assert oracle.apply_srq(3.5, 1) == 4
    assert oracle.apply_srq(-2.5, 1) == -2
    assert oracle.apply_srq(1000, 1) == 127
    assert oracle.apply_srq(-1000, 1) == -128
    assert oracle.apply_srq(2.5, 0) == 2.5
    # the output is rounded to float: 0.1 * 3 is not 0.3 in binary64
    assert oracle.apply_srq(0.31, 0.1) == float(np.float32(3 * 0.1))


def test_srq_signed_zeros():
    """roundTiesToEven (qat-linear.ts:142-148) is floor-based: a ratio in
    [-1/2, 0) gives floor -1 plus 1, which is +0, and a ratio of -0 gives
    floor(-0), which is -0 (then -0 times the scale stays -0); Math.min and
    Math.max keep -0 against 127 and -128."""
    def sign_bit(v):
        return np.signbit(np.float64(v))

    for v, neg in ((-0.0, True), (0.0, False), (-0.3, False), (-0.5, False), (-0.49, False), (0.4, False),
                   (-0.51, True), (-1e-300, False)):
        out = oracle.apply_srq(v, 1.0)
        assert (out == 0.0) == (abs(v) <= 0.5), (v, out)
        assert sign_bit(out) == neg, (v, out)
    # a whole row: scale 0 turns a negative dot into -0, which the output SRQ keeps
    x = np.ones(16, np.float32)
    codes = [0] * 16  # every weight -2: dot = -32
    out = oracle.qat_linear_int2(x, oracle.pack_int2_rows(codes, 1, 16), [0.0], 16, 1, 0.0, 0.02)
    assert out[0] == 0.0 and np.signbit(out[0])


def test_rejects_invalid_codes_and_shapes():
    with pytest.raises(ValueError, match="Int2 codes must be between 0 and 3"):
        oracle.pack_int2_rows([4] + [0] * 15, 1, 16)
    with pytest.raises(ValueError, match="Int2 input width must be divisible by 16"):
        oracle.pack_int2_rows([0] * 15, 1, 15)


def test_lm_head_known_answer():
    words = np.full(8 * 96, 0xAAAAAAAA, np.uint32)
    words[96:192] = 0xFFFFFFFF
    words[192:288] = 0x55555555
    scales = np.array([1, 0.5, 0.25, 1, 1, 1, 1, 1], np.float32)
    out = oracle.qat_linear_int2(np.ones(1536, np.float32), words, scales, 1536, 8)
    assert out.tolist() == [0, 768, -384, 0, 0, 0, 0, 0]
    # and with an output SRQ of scale 8: 768 -> clamp(96) * 8, -384 -> -48 * 8
    out = oracle.qat_linear_int2(np.ones(1536, np.float32), words, scales, 1536, 8, output_scale=8.0)
    assert out.tolist() == [0, 768, -384, 0, 0, 0, 0, 0]
    out = oracle.qat_linear_int2(np.ones(1536, np.float32), words, scales, 1536, 8, output_scale=4.0)
    assert out.tolist() == [0, 508, -384, 0, 0, 0, 0, 0]


def test_input_srq_and_block_major_order():
    rng = np.random.default_rng(1)
    V, D = 24, 128
    codes = rng.integers(0, 4, V * D).astype(np.uint8)
    words = oracle.pack_int2_rows(codes, V, D)
    x = rng.normal(0, 2, D).astype(np.float32)
    scales = rng.uniform(0.001, 0.01, V).astype(np.float32)
    # input SRQ by hand, then the int2 dot in the order of the columns
    q = np.array([oracle.apply_srq(float(v), 0.05) for v in x])
    want = np.array([np.float32(sum((int(codes[r * D + k]) - 2) * q[k] for k in range(D)) * float(scales[r]))
                     for r in range(V)], np.float32)
    got = oracle.qat_linear_int2(x, words, scales, D, V, input_scale=0.05)
    assert np.array_equal(got, want)
    bm = oracle.repack_block_major(words, V, D)
    wpr = D // 16
    for r in range(V):
        for b in range(D // 64):
            assert bm[(b * V + r) * 4:(b * V + r) * 4 + 4].tolist() == words[r * wpr + 4 * b:r * wpr + 4 * b + 4].tolist()
