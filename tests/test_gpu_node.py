"""GPU parity through the Node host: sampleToken / Engine.sampleRows /
constraints / lm_head called from JavaScript through the N-API addon, checked
against the oracle's JavaScript restatement of the reference sampler."""
import pytest

from test_node_host import run_node_tests

pytestmark = pytest.mark.gpu


def test_node_host_parity_on_gpu():
    out = run_node_tests("gpu_parity.js", 280)
    assert "all 13 passed" in out


def test_node_decode_loop_on_gpu():
    """The decode loop (node/session.js) against the reference's loop driven
    by the oracle sampler: tokens, stops, draw counts, log-probabilities,
    constraint and reasoning-channel behaviour."""
    out = run_node_tests("gpu_session.js", 280)
    assert "all 6 passed" in out
