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
import tempfile
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


# Columns a routed-rule TSV must name; the weight column's name is the bank's
# weight_field.  Checked in this order, so the first missing one is reported.
def _required_columns(weight_field):
    return ("head_id", "body_ids", weight_field, "group_id")


def _load_sidecar(cache_path, source, signature):
    """The sidecar's record when it is a version-1 index of ``source`` with
    the file's current signature; None when it is absent, unreadable or
    stale."""
    try:
        record = json.loads(cache_path.read_text())
    except (OSError, ValueError):
        return None
    if not isinstance(record, dict):
        return None
    fresh = (record.get("version") == 1, record.get("signature") == signature, record.get("source") == source)
    return record if all(fresh) else None


def _store_sidecar(cache_path, record):
    """Writes the record so that readers see the old sidecar or the whole
    new one: a uniquely named file beside it, then one rename over it."""
    cache_path.parent.mkdir(parents=True, exist_ok=True)
    fd, staged = tempfile.mkstemp(dir=str(cache_path.parent), prefix=cache_path.name + ".", suffix=".tmp")
    try:
        with os.fdopen(fd, "w") as out:
            json.dump(record, out)
        os.replace(staged, cache_path)
    except BaseException:
        if os.path.exists(staged):
            os.unlink(staged)
        raise


class IndexedRuleBank:
    """Byte-range index of a routed-rule TSV, read from or written to the
    JSON sidecar ``cache_path`` (rules/indexed_bank.py:21-88).  Public
    attributes as the reference's: path, weight_field, signature, columns,
    heads, index_reused, index_seconds, materialization_seconds,
    loaded_heads."""

    def __init__(self, path, cache_path, weight_field="weight"):
        clock = time.perf_counter()
        self.path = Path(path).resolve()
        self.weight_field = weight_field
        self.signature = _signature(self.path)
        self.materialization_seconds = 0.0
        self.loaded_heads = 0
        cache_path = Path(cache_path)
        record = _load_sidecar(cache_path, str(self.path), self.signature)
        self.index_reused = record is not None
        if record is None:
            record = self._index()
            _store_sidecar(cache_path, record)
        absent = [name for name in _required_columns(weight_field) if name not in record["columns"]]
        if absent:
            raise ValueError("Missing routed-rule column: %s" % absent[0])
        self.columns, self.heads = record["columns"], record["heads"]
        self.index_seconds = time.perf_counter() - clock

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

    def _rows(self):
        """(row id, fields) of every row of the head's runs in file order;
        each run must hold the number of rows its index entry records."""
        with self.bank.path.open("rb") as f:
            for start, end, first_id, count in self.blocks:
                f.seek(start)
                parsed = 0
                for fields in csv.reader(io.StringIO(f.read(end - start).decode()), delimiter="\t"):
                    yield first_id + parsed, fields
                    parsed += 1
                if parsed != count:
                    raise ValueError("Rule index row-count mismatch")

    def _materialize(self):
        """One rule per distinct body, in order of first appearance: the id
        of its first row, weight 1, and rank_weights holding its weight in
        every group 0 .. (largest group of the head).  A second row of a
        (body, group) whose first weight is nonzero is an error."""
        bank = self.bank
        pos = {name: i for i, name in enumerate(bank.columns)}
        head_col, body_col = pos["head_id"], pos["body_ids"]
        weight_col, group_col = pos[bank.weight_field], pos["group_id"]
        body_slot = {}        # body -> its rule's index
        first_row = []        # rule index -> id of the body's first row
        cell = {}             # (rule index, group) -> weight
        groups = 0
        for row_id, fields in self._rows():
            if int(fields[head_col]) != self.head:
                raise ValueError("Rule index relation mismatch")
            body = tuple(int(x) for x in fields[body_col].split())
            group = int(fields[group_col])
            if group < 0:
                raise ValueError("Negative rule group")
            weight = float(fields[weight_col])
            k = body_slot.get(body)
            if k is None:
                k = body_slot[body] = len(first_row)
                first_row.append(row_id)
            if cell.get((k, group), 0.0) != 0.0:
                raise ValueError("duplicate Horn rule/group instance")
            cell[(k, group)] = weight
            groups = max(groups, group + 1)
        return [dict(rule_id=first_row[k], head=self.head, body=body, weight=1.0, group_id=None,
                     rank_weights=tuple(cell.get((k, g), 0.0) for g in range(groups)))
                for body, k in body_slot.items()]

    def compact(self):
        """The head's compacted rules (computed once per object)."""
        if self._compact is None:
            clock = time.perf_counter()
            if _signature(self.bank.path) != self.bank.signature:
                raise RuntimeError("Rule file changed after indexing")
            self._compact = self._materialize()
            self.bank.materialization_seconds += time.perf_counter() - clock
            self.bank.loaded_heads += 1
        return self._compact
