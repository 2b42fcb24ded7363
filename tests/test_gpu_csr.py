"""The GPU CSR builder (fl_csr_build_side_gpu) against the host builder and
the oracle (csr.cpp:12-69): every array of both sides bit for bit, on the
five benchmark graphs and on edge cases."""
import numpy as np
import pytest
import torch

from flashlog_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


def _check(h, t, r, E):
    fk = _fk()
    gpu = fk.build_csr_structure(*(torch.from_numpy(np.asarray(a)).cuda() for a in (h, t, r)), E)
    host = fk.build_csr_structure(*(torch.from_numpy(np.asarray(a)) for a in (h, t, r)), E)
    assert len(gpu) == len(host) == 16
    for k, (a, b) in enumerate(zip(gpu, host)):
        assert a.is_cuda and a.dtype == b.dtype and torch.equal(a.cpu(), b), k
    return gpu


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_gpu_csr_matches_host_builder(cfg):
    h, r, t, E, R = synth.make_graph(cfg)
    gpu = _check(h, t, r, E)
    if cfg <= 3:  # and the oracle, on the smaller graphs
        for k, (a, b) in enumerate(zip(gpu, O.build_csr_structure(h, t, r, E))):
            assert np.array_equal(a.cpu().numpy(), b), k


def test_gpu_csr_edge_cases():
    rng = np.random.default_rng(0)
    # sources and destinations with gaps, duplicate triples, the largest relation id
    E = 50
    h = np.array([49, 3, 3, 3, 0, 49, 3, 17], np.int64)
    t = np.array([0, 4, 4, 5, 49, 0, 4, 17], np.int64)
    r = np.array([32767, 2, 2, 1, 0, 32767, 0, 5], np.int64)
    _check(h, t, r, E)
    _check(np.zeros(0, np.int64), np.zeros(0, np.int64), np.zeros(0, np.int64), 7)
    _check(rng.integers(0, 5, 3000), rng.integers(0, 5, 3000), rng.integers(0, 3, 3000), 5)
    fk = _fk()
    bad = [torch.tensor(x, device="cuda") for x in ([0, 5], [1, 2], [0, 0])]
    with pytest.raises(ValueError):
        fk.build_csr_structure(*bad, 5)  # source 5 outside [0, 5)
    bad = [torch.tensor(x, device="cuda") for x in ([0, 1], [1, 2], [0, 40000])]
    with pytest.raises(ValueError):
        fk.build_csr_structure(*bad, 5)  # relation above 32767


def test_gpu_rule_csr_matches_host():
    from flashlog_amd.rules import prepare as P
    h, r, t, E, R = synth.make_graph(3)
    args = [torch.from_numpy(a) for a in (h, t, r)]
    host = P.build_rule_csr_structure(*args, E)
    gpu = P.build_rule_csr_structure(*(a.cuda() for a in args), E)
    for a, b in zip(gpu, host):
        assert a.is_cuda and torch.equal(a.cpu(), b)
