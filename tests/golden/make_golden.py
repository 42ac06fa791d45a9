"""Writes the golden fixtures of this directory (run from the repository root):

    python tests/golden/make_golden.py

select_rows.npz  crafted selection rows: per case the root's child arrays, the child picked by
                 each simulation of one wave, and the visit counts after the wave
search_trees.npz small whole searches with replayed evaluator rows: every wave's paths and
                 the final tree (N, W, P, parent, row offset, row length, action)

Every expected value is computed twice, by the numpy-float32 restatement and by the C oracle
(oracle/golden.py). A case on which the two differ stops the script. The reference is never
imported: it ships no golden vectors for this path, so the fixtures are the restatements'
answers, frozen.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import golden  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def main() -> None:
    cases = golden.crafted_row_cases()
    picks, n_after = [], []
    for i, c in enumerate(cases):
        p_np, n_np = golden.crafted_expected_np(c)
        p_c, n_c = golden.crafted_expected_oracle(c)
        if not (np.array_equal(p_np, p_c) and np.array_equal(n_np, n_c)):
            raise SystemExit(f"crafted case {i} ({c['kind']}, k={c['k']}, m={c['m']}): numpy and "
                             "C oracle differ")
        picks.append(p_np)
        n_after.append(n_np)
    np.savez_compressed(os.path.join(HERE, "select_rows.npz"),
                        **golden.pack_crafted(cases, picks, n_after))
    print(f"select_rows.npz: {len(cases)} cases, {sum(len(p) for p in picks)} picks")

    out = {}
    for c in golden.SEARCH_CASES:
        r = golden.search_expected(c)
        for key, v in r.items():
            out[f"{c['name']}/{key}"] = v
        print(f"search_trees.npz: {c['name']}: {len(r['N'])} nodes, {len(r['path_len'])} paths")
    np.savez_compressed(os.path.join(HERE, "search_trees.npz"), **out)


if __name__ == "__main__":
    main()
