"""Writes the golden fixtures of tests/golden/ from the reference's own code.

Inputs are seeded random graphs; outputs come from the reference's
CUDA-free headers compiled in place (oracle/_ref/libgtann_ref.so, see
oracle/Makefile): prune_windowed_core.hpp (detour counts + selection, full
window), edge_chunk_accumulator.hpp (rank-ordered reverse merge) and
translate_graph_ids.hpp.  Run in a container that has /root/reference:

    make -C oracle && python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import gt_oracle as O  # noqa: E402


def graphs(rng):
    cases = []
    for (N, M, K, pad, dup) in [(40, 6, 3, 0.0, False), (60, 8, 4, 0.1, True), (200, 16, 8, 0.0, True),
                                (300, 64, 32, 0.02, True), (150, 96, 48, 0.0, True), (120, 32, 32, 0.0, False)]:
        if dup:
            G = rng.integers(0, N, size=(N, M)).astype(np.int32)
        else:
            G = np.stack([rng.permutation(np.delete(np.arange(N), i))[:M] for i in range(N)]).astype(np.int32)
        if pad:
            G[rng.random((N, M)) < pad] = -1
        cases.append((G, K))
    return cases


def main():
    if not O.ref_available():
        sys.exit("reference harness not built (make -C oracle with /root/reference present)")
    rng = np.random.default_rng(20261201)
    out = {}
    for c, (G, K) in enumerate(graphs(rng)):
        res, rc = O.ref_cagra_prune(G, K)
        out[f"prune{c}_G"] = G
        out[f"prune{c}_K"] = np.int32(K)
        out[f"prune{c}_rc"] = np.int32(rc)
        out[f"prune{c}_out"] = res
        out[f"prune{c}_counts0"] = O.ref_detour_counts(G, 0)
    np.savez_compressed(os.path.join(HERE, "prune_golden.npz"), **out)

    out = {}
    for c, (N, K, hub) in enumerate([(50, 6, False), (400, 32, True), (300, 48, True), (64, 8, True)]):
        F = rng.integers(0, N, size=(N, K)).astype(np.uint32)
        if hub:   # many rows pointing at node 0 and 1: in-degree far above 64
            F[rng.random((N, K)) < 0.3] = 0
            F[rng.random((N, K)) < 0.1] = 1
        out[f"rev{c}_F"] = F
        out[f"rev{c}_out"] = O.ref_reverse_merge(F)
    np.savez_compressed(os.path.join(HERE, "revmerge_golden.npz"), **out)

    out = {}
    for c, (N, K) in enumerate([(100, 8), (1000, 32)]):
        g = rng.integers(0, N, size=(N, K)).astype(np.uint32)
        inv = rng.permutation(N).astype(np.uint32)
        out[f"tr{c}_g"] = g
        out[f"tr{c}_inv"] = inv
        out[f"tr{c}_out"] = O.ref_translate(g, inv)
    np.savez_compressed(os.path.join(HERE, "translate_golden.npz"), **out)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
