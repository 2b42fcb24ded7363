"""Relation-at-a-time access to a routed-rule TSV through a byte-range index
(rules/indexed_bank.py:1-134).

The rule file is a TSV whose header names at least head_id (first column),
body_ids, the weight field and group_id; rows of one head come in runs of
consecutive lines.  The index lists, per head, every run as [first byte, end
byte, id of its first row, row count], row ids counting data rows from 0 in
file order.  It is kept in a JSON sidecar:

  {"version": 1, "source": <resolved path>, "signature": [st_dev, st_ino,
   st_size, st_mtime_ns, st_ctime_ns], "columns": [...], "heads": {"<head>":
   [[start, end, first_id, count], ...]}, "scalar_instances": <rows>}

with the reference's keys and meaning, so a sidecar written by either
implementation is reused by the other while the file's signature holds.

Indexing here is a vectorized pass over the memory-mapped bytes, a window
of whole lines at a time: the line starts (after every newline), the first
non-digit byte of each line, and the head value of the lines that start
with digits and a tab.  A run starts at every such line whose head bytes
differ from the previous such line's; a line that does not start with
digits and a tab continues the current run (as in the reference's scan; it
fails when its run is materialized).  The first data line must start a run,
and a run's head must have at most 31 digits (the reference reads it from
the line's first 32 bytes) -- and here at most 18 (heads are int64).  compact() parses a head's runs with the csv module and merges
rows with equal bodies into one rule whose rank_weights hold the weight of
every group, with the reference's checks (negative group, duplicate
(body, group), row counts, head mismatch, file changed after indexing).
"""
import csv
import io
import json
import mmap
import os
import time
from pathlib import Path

import numpy as np

_MAX_HEAD_BYTES = 32   # the reference reads a run's head from its first 32 bytes
_MAX_HEAD_DIGITS = 18  # heads are parsed as int64 (relation ids)
_WINDOW = 8 << 20      # bytes scanned per vectorized step


def _signature(path):
    s = path.stat()
    return [s.st_dev, s.st_ino, s.st_size, s.st_mtime_ns, s.st_ctime_ns]


def _scan_window(buf, lo, hi, line_starts):
    """For the lines starting at ``line_starts`` (all in [lo, hi), the window
    ending at a line end): whether each starts with digits and a tab, the
    number of digits, and their value (lines with at most 18 digits)."""
    w = buf[lo:hi]
    nondigit = np.flatnonzero((w < 48) | (w > 57)) + lo
    rel = line_starts
    k = np.searchsorted(nondigit, rel)
    q = np.where(k < nondigit.size, nondigit[np.minimum(k, max(nondigit.size - 1, 0))], hi) \
        if nondigit.size else np.full(rel.size, hi)
    length = q - rel
    qb = np.where(q < hi, buf[np.minimum(q, hi - 1)], 0) if hi > lo else np.zeros(rel.size, np.uint8)
    is_head = (length >= 1) & (q < hi) & (qb == 9)
    value = np.zeros(rel.size, np.int64)
    parse = is_head & (length <= _MAX_HEAD_DIGITS)
    idx = np.flatnonzero(parse)
    for j in range(_MAX_HEAD_DIGITS):
        sel = idx[length[idx] > j]
        if sel.size == 0:
            break
        value[sel] = value[sel] * 10 + (buf[rel[sel] + j].astype(np.int64) - 48)
    return is_head, length, value


def _head_runs(data, first):
    """([(head string, start, end, first row id, rows)], rows, error) of the
    data section data[first:], runs in file order; error is the message of
    a malformed file (returned, not raised, so that no array over the mapped
    bytes outlives this call in a traceback)."""
    n = len(data)
    if first >= n:
        return [], 0, None
    buf = np.frombuffer(data, dtype=np.uint8)
    runs = []  # (head value, start byte, first line) of every run
    prev = None  # (value, digits) of the previous line that starts with digits and a tab
    line_no = 0
    lo = first
    while lo < n:
        hi = min(n, lo + _WINDOW)
        if hi < n:  # end the window after its last newline (or extend to one)
            cut = data.rfind(b"\n", lo, hi)
            if cut < 0:
                cut = data.find(b"\n", hi)
            hi = n if cut < 0 else cut + 1
        w = buf[lo:hi]
        starts = np.concatenate(([lo], np.flatnonzero(w == 10) + lo + 1))
        starts = starts[starts < hi]
        is_head, length, value = _scan_window(buf, lo, hi, starts)
        if line_no == 0 and not (is_head[0] and length[0] < _MAX_HEAD_BYTES):
            return [], 0, "Invalid numeric rule head at byte %d" % first
        hs = np.flatnonzero(is_head)
        if hs.size:
            v, d = value[hs], length[hs]
            change = np.ones(hs.size, bool)
            change[1:] = (v[1:] != v[:-1]) | (d[1:] != d[:-1])
            if prev is not None:
                change[0] = (int(v[0]), int(d[0])) != prev
            for i in hs[change]:
                if length[i] >= _MAX_HEAD_BYTES:
                    return [], 0, "Invalid numeric rule head at byte %d" % int(starts[i])
                if length[i] > _MAX_HEAD_DIGITS:
                    return [], 0, "Rule head at byte %d has more than %d digits" % (int(starts[i]),
                                                                                    _MAX_HEAD_DIGITS)
                runs.append((int(value[i]), int(starts[i]), line_no + int(i)))
            prev = (int(v[-1]), int(d[-1]))
        line_no += starts.size
        lo = hi
    out = []
    for j, (val, start, first_line) in enumerate(runs):
        end = runs[j + 1][1] if j + 1 < len(runs) else n
        next_line = runs[j + 1][2] if j + 1 < len(runs) else line_no
        out.append((str(val), start, end, first_line, next_line - first_line))
    return out, line_no, None


class IndexedRuleBank:
    """Byte-range index of a routed-rule TSV, read from or written to the
    JSON sidecar ``cache_path`` (rules/indexed_bank.py:21-88)."""

    def __init__(self, path, cache_path, weight_field="weight"):
        started = time.perf_counter()
        self.path = Path(path).resolve()
        self.weight_field = weight_field
        self.materialization_seconds = 0.0
        self.loaded_heads = 0
        self.signature = _signature(self.path)
        cache_path = Path(cache_path)
        cached = None
        if cache_path.exists():
            try:
                cached = json.loads(cache_path.read_text())
            except (ValueError, OSError):
                cached = None
        self.index_reused = bool(cached and cached.get("version") == 1 and cached.get("signature") == self.signature
                                 and cached.get("source") == str(self.path))
        if not self.index_reused:
            cached = self._index()
            cache_path.parent.mkdir(parents=True, exist_ok=True)
            tmp = cache_path.with_name(cache_path.name + ".%d.tmp" % os.getpid())
            tmp.write_text(json.dumps(cached))
            os.replace(tmp, cache_path)
        self.columns = cached["columns"]
        for name in ("head_id", "body_ids", weight_field, "group_id"):
            if name not in self.columns:
                raise ValueError("Missing routed-rule column: %s" % name)
        self.heads = cached["heads"]
        self.index_seconds = time.perf_counter() - started

    def _index(self):
        with self.path.open("rb") as f:
            if os.fstat(f.fileno()).st_size == 0:
                raise ValueError("Rule TSV has no header newline")
            with mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as data:
                first = data.find(b"\n") + 1
                if not first:
                    raise ValueError("Rule TSV has no header newline")
                columns = next(csv.reader([data[:first].decode().strip()], delimiter="\t"))
                if columns[0] != "head_id":
                    raise ValueError("Indexed rules require head_id as the first column")
                runs, rows, error = _head_runs(data, first)
        if error:
            raise ValueError(error)
        heads = {}
        for head, lo, hi, first_id, count in runs:
            heads.setdefault(head, []).append([lo, hi, first_id, count])
        if _signature(self.path) != self.signature:
            raise RuntimeError("Rule file changed while indexing")
        return dict(version=1, source=str(self.path), signature=self.signature, columns=columns, heads=heads,
                    scalar_instances=rows)

    def get(self, head, default=None):
        blocks = self.heads.get(str(head))
        return IndexedHeadRules(self, int(head), blocks) if blocks else default


class IndexedHeadRules:
    """The rules of one head, materialized on demand
    (rules/indexed_bank.py:91-134)."""

    def __init__(self, bank, head, blocks):
        self.bank, self.head, self.blocks = bank, head, blocks
        self._compact = None

    def __len__(self):
        return sum(b[3] for b in self.blocks)

    def compact(self):
        """One rule per distinct body (first row's id), weight 1, its
        rank_weights the weight of every group 0..max group of the head."""
        if self._compact is not None:
            return self._compact
        started = time.perf_counter()
        bank = self.bank
        if _signature(bank.path) != bank.signature:
            raise RuntimeError("Rule file changed after indexing")
        col = {name: i for i, name in enumerate(bank.columns)}
        ih, ib, iw, ig = col["head_id"], col["body_ids"], col[bank.weight_field], col["group_id"]
        merged = {}  # body -> [first rule id, {group: weight}]
        width = 0
        with bank.path.open("rb") as f:
            for start, end, first_id, count in self.blocks:
                f.seek(start)
                text = f.read(end - start).decode()
                seen = 0
                for offset, row in enumerate(csv.reader(io.StringIO(text), delimiter="\t")):
                    if int(row[ih]) != self.head:
                        raise ValueError("Rule index relation mismatch")
                    body = tuple(int(x) for x in row[ib].split())
                    group = int(row[ig])
                    if group < 0:
                        raise ValueError("Negative rule group")
                    weight = float(row[iw])
                    width = max(width, group + 1)
                    slot = merged.setdefault(body, [first_id + offset, {}])
                    if slot[1].get(group, 0.0) != 0.0:
                        raise ValueError("duplicate Horn rule/group instance")
                    slot[1][group] = weight
                    seen += 1
                if seen != count:
                    raise ValueError("Rule index row-count mismatch")
        self._compact = [dict(rule_id=rid, head=self.head, body=body, weight=1.0, group_id=None,
                              rank_weights=tuple(w.get(g, 0.0) for g in range(width)))
                         for body, (rid, w) in merged.items()]
        bank.materialization_seconds += time.perf_counter() - started
        bank.loaded_heads += 1
        return self._compact
