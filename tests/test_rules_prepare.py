"""The rule-serving CSR and its cache file (rules/prepare.py:29-134,230-232):
the fields against the oracle's CSR, the edge order against the reference's
own key argsort on a graph large enough for torch's stable sort path, the
cache round trip, and the head helpers."""
import numpy as np
import pytest
import torch

from flashlog_amd.rules import prepare as P
from flashlog_amd.rules.evaluate import CSR_RULE_FIELDS
from oracle import oracle as O


def _graph(seed, E, R, M):
    rng = np.random.default_rng(seed)
    return rng.integers(0, E, M), rng.integers(0, R, M), rng.integers(0, E, M)


def test_rule_csr_fields_match_oracle(tmp_path):
    h, r, t = _graph(0, 300, 7, 5000)
    csr = P.build_rule_csr_structure(torch.from_numpy(h), torch.from_numpy(t), torch.from_numpy(r), 300)
    want = O.build_csr_structure(h, t, r, 300)
    assert len(csr) == 16
    for i, x in enumerate(csr):
        if i in CSR_RULE_FIELDS:
            assert np.array_equal(x.numpy(), want[i]), i
        else:
            assert x.numel() == 0, i
    path = P.write_rule_csr(tmp_path / "c" / "train_compact_csr.pt", csr, 300)
    n, back = P.read_rule_csr(path)
    assert n == 300 and all(torch.equal(a, b) for a, b in zip(csr, back))


def test_rule_csr_order_matches_reference_argsort():
    """Above 32767 edges torch's CPU argsort of int64 keys is stable, so the
    reference's ordering (rules/prepare.py:75-82) equals edge order within
    equal (source, relation) keys; the columns agree."""
    h, r, t = _graph(1, 2000, 5, 40000)
    csr = P.build_rule_csr_structure(torch.from_numpy(h), torch.from_numpy(t), torch.from_numpy(r), 2000)
    th, tr, tt = (torch.from_numpy(a) for a in (h, r, t))
    base = int(tr.max()) + 1
    for rows, cols, field in ((th, tt, 1), (tt, th, 5)):
        order = (rows * base + tr).argsort()
        assert torch.equal(csr[field], cols[order].to(torch.int32))


def test_head_helpers(tmp_path):
    f = tmp_path / "heads.txt"
    f.write_text("5\n\n1\n 3 \n")
    assert P.read_heads(f, 3) == [1, 3, 5]
    f.write_text("1\n1\n")
    with pytest.raises(ValueError, match="duplicate"):
        P.read_heads(f, 3)
    f.write_text("6\n")
    with pytest.raises(ValueError, match="invalid directed"):
        P.read_heads(f, 3)
    assert P.directed_heads_from_train_relations(np.array([2, 0, 2, 4], np.int32), 6) == [0, 2, 4, 6, 8, 10]
    assert P.directed_heads_from_train_relations(np.array([], np.int64), 6) == []
    with pytest.raises(ValueError, match="invalid base relation"):
        P.directed_heads_from_train_relations(np.array([6]), 6)


def test_load_train_columns(tmp_path):
    f = tmp_path / "train_id.txt"
    f.write_text("0\t1\t2\n3\t0\t1\n")
    (s, r, t), parser = P.load_train_columns(f)
    assert s.tolist() == [0, 3] and r.tolist() == [1, 0] and t.tolist() == [2, 1] and s.dtype == np.int32
    assert parser in ("pyarrow-csv-parallel", "pandas-c")
