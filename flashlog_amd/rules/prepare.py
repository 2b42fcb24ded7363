"""The rule-serving training CSR and its cache file (rules/prepare.py:29-94,
230-232).

build_rule_csr_structure gives the propagation 16-tuple with only the fields
rule grounding reads: the columns (1, 5) and the group arrays (8-15) of both
sides; the row pointers, edge relations and sort permutations (0, 2-4, 6,
7) are empty tensors.  Within a source row the edges are ordered by
relation, equal (source, relation) neighbours in edge order, which seeded
walks depend on.  The reference orders them with torch's CPU argsort of
source * (max relation + 1) + relation: for graphs of 32768 edges and more
that sort is stable (its radix path) and the orders agree; below that size
torch leaves the order of equal keys open.

write_rule_csr / read_rule_csr hold the cache file train_compact_csr.pt:
a torch file {"num_entities": E, "csr": <the tuple, CPU tensors>}, read
with weights_only=True.
"""
from pathlib import Path

import numpy as np
import torch

from ..flashlog_kernel import flashlog_kernel as fk
from .evaluate import CSR_RULE_FIELDS


def read_heads(path, num_relations):
    """Sorted directed query heads, one integer per nonblank line; duplicates
    and heads outside [0, 2 * num_relations) are errors
    (rules/prepare.py:29-37)."""
    heads = sorted(int(line) for line in Path(path).read_text().splitlines() if line.strip())
    if len(set(heads)) != len(heads):
        raise ValueError("query-head file contains duplicate relations")
    if heads and (heads[0] < 0 or heads[-1] >= 2 * num_relations):
        raise ValueError("query-head file contains an invalid directed relation")
    return heads


def directed_heads_from_train_relations(relations, num_relations):
    """Every base relation present in the training relations, ascending,
    then the same relations offset by num_relations (rules/prepare.py:40-59)."""
    values = np.asarray(relations)
    if values.size:
        lo, hi = values.min(), values.max()
        if lo < 0 or hi >= num_relations:
            raise ValueError("Train contains an invalid base relation")
    base = np.unique(values)
    return np.concatenate((base, base + num_relations)).tolist()


def build_rule_csr_structure(row_indices, col_indices, r_indices, num_nodes):
    """The rule-serving CSR (rules/prepare.py:62-94) on the inputs' device:
    built on the GPU for device inputs (fl_csr_build_side_gpu), by the
    library's host builder for CPU inputs; the same arrays either way."""
    csr = fk.build_csr_structure(row_indices, col_indices, r_indices, int(num_nodes))
    return tuple(x if i in CSR_RULE_FIELDS else torch.empty(0, device=x.device) for i, x in enumerate(csr))


def load_train_columns(path):
    """(source, relation, target) int32 columns of a three-column
    tab-separated file, and the parser used (rules/prepare.py:97-134)."""
    try:
        import pyarrow as pa
        import pyarrow.csv as pcsv
    except ImportError:
        import pandas as pd
        frame = pd.read_csv(path, sep="\t", header=None, engine="c", dtype={0: np.int32, 1: np.int32, 2: np.int32})
        return tuple(frame[c].to_numpy(copy=False) for c in range(3)), "pandas-c"
    names = ("source", "relation", "target")
    table = pcsv.read_csv(path, read_options=pcsv.ReadOptions(column_names=names, block_size=8 << 20,
                                                              use_threads=True),
                          parse_options=pcsv.ParseOptions(delimiter="\t"),
                          convert_options=pcsv.ConvertOptions(column_types={n: pa.int32() for n in names}))
    return tuple(table.column(n).combine_chunks().to_numpy(zero_copy_only=True) for n in names), \
        "pyarrow-csv-parallel"


def write_rule_csr(path, csr, num_entities):
    """train_compact_csr.pt (rules/prepare.py:230-232)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    torch.save({"num_entities": int(num_entities), "csr": tuple(x.detach().cpu() for x in csr)}, path)
    return path


def read_rule_csr(path, device="cpu"):
    """(num_entities, csr) of a train_compact_csr.pt, the rule fields moved
    to ``device``."""
    payload = torch.load(path, map_location="cpu", weights_only=True)
    csr = tuple(t.to(device) if i in CSR_RULE_FIELDS else torch.empty(0, device=device)
                for i, t in enumerate(payload["csr"]))
    return int(payload["num_entities"]), csr
