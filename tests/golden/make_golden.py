"""Writes the golden fixtures for the dense hop from the reference's own CPU
code (flashlog.cpp and csr.cpp compiled in place into oracle/_ref by
oracle/Makefile.ref), plus the reference's public API surface (names and
parameter lists, parsed from flashlog_kernel/flashlog_kernel.py with ast).

Run in the container that has /root/reference:
    make -f oracle/Makefile.ref && python tests/golden/make_golden.py
Outputs tests/golden/dense_golden.npz and tests/golden/api_surface.json.
"""
import ast
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle", "_ref"))
REF = "/root/reference"

import flashlog_csr_ref as csr_ref  # noqa: E402
import flashlog_ref_cpp as ref  # noqa: E402


def graph(seed, E, R, M):
    rng = np.random.default_rng(seed)
    h = rng.integers(0, E, M)
    t = rng.integers(0, E, M)
    r = rng.integers(0, R, M)
    # a few hubs and duplicate edges to exercise groups and quotas
    h[: M // 5] = rng.integers(0, 3, M // 5)
    dup = rng.integers(0, M, M // 20)
    h[-dup.size:], t[-dup.size:], r[-dup.size:] = h[dup], t[dup], r[dup]
    return h.astype(np.int64), r.astype(np.int64), t.astype(np.int64)


def main():
    cases = {}
    specs = [(0, 60, 3, 400, 4, 3, [1 << 60, 1, 3, 5]),
             (1, 150, 5, 900, 2, 3, [1 << 60, 2, 7]),
             (2, 40, 2, 300, 3, 1, [1 << 60, 4])]
    for seed, E, R, M, B, L, Ks in specs:
        h, r, t = graph(seed, E, R, M)
        o = csr_ref.build_side(h, t, r, E)
        i = csr_ref.build_side(t, h, r, E)
        csr = [np.asarray(a) for a in (*o[:4], *i[:4], *o[4:], *i[4:])]
        rng = np.random.default_rng(100 + seed)
        BL, n = B * L, 2 * R + 1
        A = np.zeros((BL, E), np.float32)
        for row in range(BL):
            k = rng.integers(1, E // 3)
            idx = rng.choice(E, k, replace=False)
            vals = rng.integers(1, 5, k).astype(np.float32) / 4 if row % 2 else rng.random(k).astype(np.float32)
            A[row, idx] = vals
        logits = rng.standard_normal((BL, n)).astype(np.float32)
        w = np.exp(logits) / np.exp(logits).sum(-1, keepdims=True)
        w = w.astype(np.float32)
        w[0, :R] = w[0, 0]  # equal relation weights: tie quotas
        mask = (rng.random(M) > 0.15)
        om, im = mask[csr[3]].astype(np.float32), mask[csr[7]].astype(np.float32)
        g = [rng.standard_normal((BL, E)).astype(np.float32) for _ in range(3)]
        act = np.nonzero((A != 0).any(0))[0].astype(np.int64)
        T = lambda x: torch.from_numpy(np.ascontiguousarray(x))
        base = "s%d" % seed
        cases[base + "_h"], cases[base + "_r"], cases[base + "_t"] = h, r, t
        cases[base + "_A"], cases[base + "_w"], cases[base + "_mask"] = A, w, mask
        cases[base + "_gind"], cases[base + "_gori"], cases[base + "_ginv"] = g
        for k, a in enumerate(csr):
            cases["%s_csr%d" % (base, k)] = a
        for K in Ks:
            for wot_i in (False, True):
                fo = ref.flashlog_forward_cpu(T(A), T(w), T(act), T(csr[1]), T(om), T(csr[8]), T(csr[9]), T(csr[10]),
                                              T(csr[11]), T(csr[5]), T(im), T(csr[12]), T(csr[13]), T(csr[14]),
                                              T(csr[15]), R, wot_i, K)
                bo = ref.flashlog_backward_cpu(T(g[0]), T(g[1]), T(g[2]), T(A), T(w), T(act), T(csr[1]), T(om),
                                               T(csr[8]), T(csr[9]), T(csr[10]), T(csr[11]), T(csr[5]), T(im),
                                               T(csr[12]), T(csr[13]), T(csr[14]), T(csr[15]), R, wot_i, K)
                key = "%s_K%d_w%d" % (base, min(K, 10 ** 9), int(wot_i))
                for nm, x in zip(("ind", "ori", "inv", "gA", "gw"), (*fo, *bo)):
                    cases[key + "_" + nm] = x.numpy()
    cases["specs"] = np.array([[s[0], s[1], s[2], s[3], s[4], s[5]] for s in specs], np.int64)
    np.savez_compressed(os.path.join(HERE, "dense_golden.npz"), **cases)

    write_api_surface()
    print("wrote", len(cases), "arrays")


def write_api_surface():
    """Signatures (names and parameter names only) of the reference's
    operator module and rule-scoring entry points, parsed with ast."""
    src = open(os.path.join(REF, "flashlog_kernel", "flashlog_kernel.py")).read()
    tree = ast.parse(src)
    surface = {}
    for node in tree.body:
        if isinstance(node, ast.FunctionDef):
            surface[node.name] = [a.arg for a in node.args.args]
        elif isinstance(node, ast.ClassDef):
            for sub in node.body:
                if isinstance(sub, ast.FunctionDef) and sub.name in ("forward", "backward"):
                    surface["%s.%s" % (node.name, sub.name)] = [a.arg for a in sub.args.args]
    json.dump(surface, open(os.path.join(HERE, "api_surface.json"), "w"), indent=1, sort_keys=True)
    rules = {}
    for mod in ("shared_inference", "max_inference"):
        tree = ast.parse(open(os.path.join(REF, "rules", mod + ".py")).read())
        for node in tree.body:
            if isinstance(node, ast.FunctionDef) and node.name == "score":
                rules["%s.score" % mod] = [a.arg for a in node.args.args]
    # rule evaluation primitives and scorer (rules/evaluate.py), less its CLI and file readers
    tree = ast.parse(open(os.path.join(REF, "rules", "evaluate.py")).read())
    for node in tree.body:
        if isinstance(node, ast.FunctionDef) and node.name not in ("main", "parse_args", "load_triples",
                                                                     "dictionary_size"):
            rules["evaluate.%s" % node.name] = [a.arg for a in node.args.args]
    # extraction post-processing, the rule-serving CSR and the indexed rule bank
    wanted = {"extract": ("_three_step_weights", "collapsed_rule_weights", "attention_rank_weights",
                          "fallback_rule_scores", "select_and_annotate_array", "output_lines", "output_rule_lines"),
              "prepare": ("read_heads", "directed_heads_from_train_relations", "build_rule_csr_structure",
                          "load_train_columns"),
              "indexed_bank": ("IndexedRuleBank", "IndexedHeadRules")}
    for mod, names in wanted.items():
        tree = ast.parse(open(os.path.join(REF, "rules", mod + ".py")).read())
        for node in tree.body:
            if isinstance(node, ast.FunctionDef) and node.name in names:
                rules["%s.%s" % (mod, node.name)] = [a.arg for a in node.args.args]
            elif isinstance(node, ast.ClassDef) and node.name in names:
                for sub in node.body:
                    if isinstance(sub, ast.FunctionDef) and sub.name == "__init__":
                        rules["%s.%s" % (mod, node.name)] = [a.arg for a in sub.args.args][1:]
    json.dump(rules, open(os.path.join(HERE, "rules_surface.json"), "w"), indent=1, sort_keys=True)
    # evaluation consumers of the driver (src/main.py:117-512)
    evaluation = {}
    names = ("create_eval_filter_csr", "_build_filter_edge_lookup", "_filter_csr_cache_key",
             "_build_filter_side_lookup", "_get_filter_csr_lookup", "_expand_filter_side",
             "build_filter_indices_csr", "_filter_indices_from_lookup", "build_filter_indices_graph",
             "_sparse_truth_scores", "calculate_raw_hits_sparse", "calculate_hits_full_sparse",
             "calculate_hits_full_with_filter_indices")
    tree = ast.parse(open(os.path.join(REF, "src", "main.py")).read())
    for node in tree.body:
        if isinstance(node, ast.FunctionDef) and node.name in names:
            evaluation[node.name] = [a.arg for a in node.args.args]
    json.dump(evaluation, open(os.path.join(HERE, "evaluation_surface.json"), "w"), indent=1, sort_keys=True)
    grounding = {}
    tree = ast.parse(open(os.path.join(REF, "flashlog_kernel", "soft_grounding_kernel",
                                       "soft_grounding_kernel.py")).read())
    for node in tree.body:
        if isinstance(node, ast.FunctionDef) and not node.name.startswith("_"):
            grounding[node.name] = [a.arg for a in node.args.args]
    json.dump(grounding, open(os.path.join(HERE, "grounding_surface.json"), "w"), indent=1, sort_keys=True)
    print("wrote", len(surface) + len(rules) + len(evaluation) + len(grounding), "signatures")


if __name__ == "__main__":
    if "--api-only" in sys.argv:
        write_api_surface()
    else:
        main()
