"""The routed-rule TSV byte-range index (rules/indexed_bank.py:1-134):
the index against a line-by-line scan of the file, the sidecar's reuse and
invalidation, compact() against the eager loader followed by the routed
compaction (rules/evaluate.py:63-119), and the reference's error cases."""
import json
import os

import numpy as np
import pytest

from flashlog_amd.rules import evaluate as ev
from flashlog_amd.rules import indexed_bank as ib


def _write_bank(path, rng, heads=(3, 12, 7, 3, 105, 7), rows_per=(5, 1, 9, 2, 30, 4), trailing_newline=True,
                extra_cols=True):
    cols = ["head_id", "body_ids", "weight", "group_id"] + (["confidence", "rank_weights"] if extra_cols else [])
    lines = ["\t".join(cols)]
    seen = set()
    for h, n in zip(heads, rows_per):
        for _ in range(n):
            while True:
                body = " ".join(str(x) for x in rng.integers(0, 20, rng.integers(0, 4)))
                g = int(rng.integers(0, 4))
                if (h, body, g) not in seen:
                    seen.add((h, body, g))
                    break
            w = float(rng.choice([0.0, 0.125, 0.3, 1.0 / 3.0, 2.5]))
            row = [str(h), body, repr(w), str(g)] + (["%.3f" % rng.random(), "0.1 0.2"] if extra_cols else [])
            lines.append("\t".join(row))
    text = "\n".join(lines) + ("\n" if trailing_newline else "")
    path.write_text(text)
    return text


def _scan(text):
    """Line-by-line index: runs of consecutive lines with equal head bytes."""
    header, _, body = text.partition("\n")
    pos = len(header) + 1
    heads, runs, row = {}, [], 0
    for line in body.splitlines(keepends=True):
        head = line.split("\t", 1)[0]
        if runs and runs[-1][0] == head:
            runs[-1][2] = pos + len(line)
            runs[-1][4] += 1
        else:
            runs.append([head, pos, pos + len(line), row, 1])
        pos += len(line)
        row += 1
    for head, lo, hi, first, count in runs:
        heads.setdefault(str(int(head)), []).append([lo, hi, first, count])
    return heads, row


@pytest.mark.parametrize("trailing", [True, False])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_index_matches_line_scan(tmp_path, seed, trailing):
    rng = np.random.default_rng(seed)
    path = tmp_path / "rules.tsv"
    text = _write_bank(path, rng, trailing_newline=trailing)
    bank = ib.IndexedRuleBank(path, tmp_path / "idx" / "rules.head-index.json")
    heads, rows = _scan(text)
    assert bank.heads == heads and not bank.index_reused
    side = json.loads((tmp_path / "idx" / "rules.head-index.json").read_text())
    assert list(side) == ["version", "source", "signature", "columns", "heads", "scalar_instances"]
    assert side["version"] == 1 and side["scalar_instances"] == rows and side["source"] == str(path.resolve())
    assert len(bank.get(3)) == 7 and bank.get(999) is None and bank.get(4, "x") == "x"


def test_index_windows(tmp_path, monkeypatch):
    """Windows that end mid-file give the same index as one window."""
    rng = np.random.default_rng(5)
    path = tmp_path / "rules.tsv"
    heads = tuple(int(x) for x in rng.integers(0, 50, 200))
    text = _write_bank(path, rng, heads=heads, rows_per=tuple(int(x) for x in rng.integers(1, 6, 200)))
    want, rows = _scan(text)
    for window in (64, 97, 1000):
        monkeypatch.setattr(ib, "_WINDOW", window)
        runs, n, err = ib._head_runs(text.encode(), text.index("\n") + 1)
        assert err is None
        got = {}
        for h, lo, hi, first, count in runs:
            got.setdefault(h, []).append([lo, hi, first, count])
        assert got == want and n == rows, window


def test_sidecar_reuse_and_invalidation(tmp_path):
    rng = np.random.default_rng(1)
    path = tmp_path / "rules.tsv"
    _write_bank(path, rng)
    side = tmp_path / "rules.head-index.json"
    a = ib.IndexedRuleBank(path, side)
    b = ib.IndexedRuleBank(path, side)
    assert not a.index_reused and b.index_reused and a.heads == b.heads
    # a changed file is indexed again
    _write_bank(path, np.random.default_rng(2), heads=(1, 2), rows_per=(3, 3))
    c = ib.IndexedRuleBank(path, side)
    assert not c.index_reused and set(c.heads) == {"1", "2"}
    # a corrupt sidecar is rebuilt
    side.write_text("{not json")
    assert not ib.IndexedRuleBank(path, side).index_reused
    # materializing after the file changed fails
    bank = ib.IndexedRuleBank(path, side)
    os.utime(path, ns=(1, 1))
    with pytest.raises(RuntimeError):
        bank.get(1).compact()


@pytest.mark.parametrize("seed", [0, 3, 4])
def test_compact_matches_eager_loader(tmp_path, seed):
    rng = np.random.default_rng(seed)
    path = tmp_path / "rules.tsv"
    _write_bank(path, rng)
    bank = ib.IndexedRuleBank(path, tmp_path / "s.json")
    eager = ev.load_rules(path)
    for head in {r["head"] for r in eager}:
        rules = bank.get(head)
        got = rules.compact()
        want = ev.compact_routed_rules([r for r in eager if r["head"] == head])
        assert [(r["rule_id"], r["head"], r["body"], r["weight"], r["group_id"], r["rank_weights"]) for r in got] == \
            [(r["rule_id"], r["head"], r["body"], r["weight"], r["group_id"], r["rank_weights"]) for r in want]
        assert ev.compact_routed_rules(rules) is got  # materialized once per head object
    assert bank.loaded_heads == len({r["head"] for r in eager})


def test_errors(tmp_path):
    p = tmp_path / "r.tsv"
    s = tmp_path / "s.json"
    p.write_text("")
    with pytest.raises(ValueError, match="header newline"):
        ib.IndexedRuleBank(p, s)
    p.write_text("head_id\tbody_ids\tweight\tgroup_id")
    with pytest.raises(ValueError, match="header newline"):
        ib.IndexedRuleBank(p, s)
    p.write_text("body_ids\thead_id\tweight\tgroup_id\n1\t2\t0.5\t0\n")
    with pytest.raises(ValueError, match="first column"):
        ib.IndexedRuleBank(p, s)
    p.write_text("head_id\tbody_ids\tweight\tgroup_id\nx1\t2\t0.5\t0\n")
    with pytest.raises(ValueError, match="Invalid numeric rule head"):
        ib.IndexedRuleBank(p, s)
    p.write_text("head_id\tbody_ids\tweight\tgroup_id\n1\t2\t0.5\t0\n" + "9" * 40 + "\t2\t0.5\t0\n")
    with pytest.raises(ValueError, match="Invalid numeric rule head"):
        ib.IndexedRuleBank(p, s)
    p.write_text("head_id\tbody_ids\tweight\n1\t2\t0.5\n")
    with pytest.raises(ValueError, match="Missing routed-rule column: group_id"):
        ib.IndexedRuleBank(p, s)
    p.write_text("head_id\tbody_ids\tweight\tgroup_id\n1\t2\t0.5\t-1\n")
    with pytest.raises(ValueError, match="Negative rule group"):
        ib.IndexedRuleBank(p, s).get(1).compact()
    p.write_text("head_id\tbody_ids\tweight\tgroup_id\n1\t2\t0.5\t0\n1\t2\t0.25\t0\n")
    with pytest.raises(ValueError, match="duplicate Horn rule"):
        ib.IndexedRuleBank(p, s).get(1).compact()
    # a zero weight does not block a later instance of the same (body, group)
    p.write_text("head_id\tbody_ids\tweight\tgroup_id\n1\t2\t0.0\t1\n1\t2\t0.25\t1\n")
    assert ib.IndexedRuleBank(p, s).get(1).compact()[0]["rank_weights"] == (0.0, 0.25)
    # a malformed line inside a run fails when that head is materialized
    p.write_text("head_id\tbody_ids\tweight\tgroup_id\n1\t2\t0.5\t0\n\n1\t3\t0.5\t0\n")
    bank = ib.IndexedRuleBank(p, s)
    assert bank.heads == {"1": [[p.read_text().index("\n") + 1, len(p.read_text()), 0, 3]]}
    with pytest.raises((ValueError, IndexError)):
        bank.get(1).compact()
    # header only: an empty index
    p.write_text("head_id\tbody_ids\tweight\tgroup_id\n")
    bank = ib.IndexedRuleBank(p, s)
    assert bank.heads == {} and json.loads(s.read_text())["scalar_instances"] == 0
