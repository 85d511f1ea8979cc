import os
import shutil
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gemma-webgpu-engine_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libgsample.so")


NODE = shutil.which("node")


@pytest.fixture(scope="session")
def node():
    if NODE is None:
        pytest.skip("node is not installed")
    return NODE


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.build()
    return o


@pytest.fixture(scope="session")
def sampler():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    import gsample

    s = gsample.Sampler(vocab_size=262144, max_rows=1024)
    yield s
    s.close()


@pytest.fixture(scope="session")
def synthetic_constraint(oracle):
    """The constrained workload's synthetic vocabulary (262144 byte strings)
    and 64-state DFA, with the oracle's own legal-token masks for every state
    (uint32 words, bit i of word w = id 32 w + i)."""
    import gsample

    W = gsample.workloads
    offsets, data = W.synthetic_vocab()
    nxt, finals = W.synthetic_dfa()
    viable = oracle.viable_states(nxt, finals)
    masks = np.stack([oracle.dfa_legal_mask(nxt, viable, offsets, data, s) for s in range(nxt.shape[0])])
    return offsets, data, nxt, finals, masks
