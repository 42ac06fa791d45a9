"""Known-answer cases for the selection chain and small whole searches.

TEST INFRASTRUCTURE ONLY (tests/ and tests/golden/make_golden.py).

Two kinds of case:

* **Crafted rows.** A root with k unexpanded children whose N, W and P are chosen to stress the
  selection. The cases include exact ties, priors one ulp apart, unvisited children at high
  indices, |Q| above 1e8, negative priors, c_puct = 0, VL = 0 and fractional VL. The root
  takes m simulations of one wave. Each simulation's path is [root, child], so the expected
  output is the child picked by each of the m simulations, plus the visit counts after the
  wave. The answer follows select_path / select_best_child_nogil
  (python/mcts/cpu/cython_tree_optimized.pyx:177-202,421-464).
* **Small searches.** Whole searches on tiny boards, with evaluator rows (policy, value) drawn
  from a seeded generator and replayed. The expected output is every wave's paths and the
  final tree (optimized_wave_search.py:299-483 for expansion and backup).

Both kinds are computed twice, by the numpy-float32 restatement (oracle/ref_np.py) and by the
C oracle (oracle/tree_oracle.c). The fixture generator refuses to write a case on which the two
differ.
"""
from __future__ import annotations

import json

import numpy as np

from omoknuni_quantum_amd.synthetic import games

from . import ref_np
from .oracle import Oracle

F32 = np.float32


def model_from_name(name: str) -> games.GameModel:
    kind, _, arg = name.partition(":")
    if kind == "gomoku":
        return games.gomoku(int(arg))
    if kind == "go":
        return games.go(int(arg))
    if kind == "sparse":
        return games.chess_sparse()
    raise ValueError(name)


# ---- crafted rows -----------------------------------------------------------------------

def _model_for_width(k: int) -> str:
    for bound, name in ((45, "sparse"), (121, "gomoku:11"), (169, "gomoku:13"), (225, "gomoku:15"),
                        (362, "go:19"), (441, "gomoku:21")):
        if k <= bound:
            return name
    raise ValueError(k)


def crafted_row_cases(seed: int = 2024) -> list[dict]:
    """The crafted-row cases: dicts with model, k, m, c, vl, N0 and the child arrays N, W, P."""
    rng = np.random.default_rng(seed)
    cases = []

    def add(kind, k, m, c=1.4, vl=3.0, N0=None, Nc=None, Wc=None, Pc=None, model=None):
        if Nc is None:
            Nc = rng.integers(0, 40, k)
        Nc = np.asarray(Nc, np.int32)
        if Wc is None:
            Wc = (Nc * rng.uniform(-1, 1, k)).astype(F32)
        if Pc is None:
            Pc = rng.dirichlet([0.3] * k).astype(F32)
        if N0 is None:
            N0 = int(Nc.sum()) + 1
        cases.append({"kind": kind, "model": model or _model_for_width(k), "k": int(k),
                      "m": int(m), "c": float(F32(c)), "vl": float(vl), "N0": int(N0),
                      "N": Nc.astype(np.int32), "W": np.asarray(Wc, F32),
                      "P": np.asarray(Pc, F32)})

    # random rows of every chain width, with a few unvisited children
    for k, m in ((1, 5), (3, 9), (20, 64), (45, 130), (64, 65), (65, 200), (121, 256),
                 (128, 129), (169, 300), (200, 256), (225, 512), (300, 700), (362, 1024),
                 (441, 600)):
        add("random", k, m)
    # all visited: the chain runs on scores only from the first step
    for k, m in ((40, 256), (225, 256), (362, 1024)):
        add("visited", k, m, Nc=rng.integers(1, 30, k))
    # exact ties everywhere: identical children, every step a tie broken by index
    for k, m in ((8, 40), (64, 128), (225, 300)):
        add("ties", k, m, Nc=np.full(k, 5), Wc=np.full(k, 1.25, F32), Pc=np.full(k, 1.0 / k, F32))
    # priors one ulp apart, equal N and W: the approximate scores cannot separate the children
    for k, m in ((30, 90), (200, 256)):
        p = F32(0.01)
        Pc = np.array([np.nextafter(p, F32(1), dtype=F32) if j % 3 == 1 else p for j in range(k)],
                      F32)
        add("ulp", k, m, Nc=np.full(k, 7), Wc=np.full(k, -0.5, F32), Pc=Pc)
    # values one ulp apart
    for k, m in ((50, 100),):
        w0 = F32(0.75)
        Wc = np.array([np.nextafter(w0, F32(2), dtype=F32) if j % 4 == 2 else w0 for j in range(k)],
                      F32)
        add("ulpW", k, m, Nc=np.full(k, 3), Wc=Wc, Pc=np.full(k, F32(1.0 / k), F32))
    # unvisited children only at high indices (first unvisited rule late in the row)
    for k, m in ((60, 64), (225, 64), (362, 128)):
        Nc = rng.integers(1, 20, k)
        Nc[[k - 1, k - 3]] = 0
        add("late_unvisited", k, m, Nc=Nc)
    # all unvisited
    add("all_unvisited", 100, 150, Nc=np.zeros(100, np.int64), Wc=np.zeros(100, F32))
    # |Q| beyond 1e8: every step compares exactly
    for k, m in ((40, 80), (225, 256)):
        Nc = rng.integers(1, 9, k)
        add("bigQ", k, m, Nc=Nc, Wc=(rng.uniform(-1, 1, k) * 1e12).astype(F32))
    # negative priors: exact comparison as well
    for k, m in ((40, 80), (150, 200)):
        Pc = rng.uniform(-0.02, 0.05, k).astype(F32)
        add("negP", k, m, Pc=Pc, Nc=rng.integers(1, 9, k))
    # c_puct = 0: pure value ranking with ties among equal Q
    add("c0", 64, 100, c=0.0, Nc=np.full(64, 4), Wc=np.round(rng.uniform(-4, 4, 64)).astype(F32))
    # large c_puct
    add("c50", 225, 256, c=50.0)
    # VL = 0 (every rank takes the first rank's choice), VL = 1, fractional VL = 2.5
    add("vl0", 225, 64, vl=0.0)
    add("vl0_np0", 10, 5, vl=0.0, N0=0)
    add("vl1", 100, 256, vl=1.0)
    add("vl2.5", 225, 256, vl=2.5)
    # single members under each narrow kernel (per-lane best-child scan) and under wide kernels
    for k in (1, 17, 45, 100, 160, 225, 362):
        add("single", k, 1)
    # narrow rows under the wide kernels
    add("narrow_in_wide", 30, 200, model="gomoku:15")
    add("narrow_in_go", 64, 300, model="go:19")
    add("small_in_8", 100, 130, model="gomoku:21")
    # NaN values of either sign (a NaN score is never a pick: every comparison with it is
    # false), in rows held one per lane, in windows and in wide rows
    nan_pos = np.array([0x7FC00000], np.uint32).view(F32)[0]
    nan_neg = np.array([0xFFC00000], np.uint32).view(F32)[0]
    for k, m, nan in ((40, 100, nan_pos), (63, 100, nan_neg), (225, 256, nan_pos),
                      (362, 300, nan_neg)):
        Nc = rng.integers(1, 20, k)
        Wc = (Nc * rng.uniform(-1, 1, k)).astype(F32)
        Wc[rng.choice(k, 3, replace=False)] = nan
        add("nanW", k, m, Nc=Nc, Wc=Wc)
    for c in pinned_row_cases():
        c = dict(c)
        c.update(N=np.asarray(c["N"], np.int32), W=np.asarray(c["W"], F32),
                 P=np.asarray(c["P"], F32))
        cases.append(c)
    return cases


# ---- pinned rows --------------------------------------------------------------------------
# Rows built by hand so that one plausible misreading of select_best_child_nogil /
# select_path (cython_tree_optimized.pyx:177-202,436-461) picks another child than the rule
# does.  The rule: Np = N0 + VL (the arriving simulation's virtual loss is added first); the
# first child with N == 0 wins; otherwise the strict argmax of
#     W / ((float)N + VL) + ((c * P) * sqrt((float)Np)) / (float)(1 + N)
# in float32, source order, lowest index on ties; children carry the virtual loss of earlier
# simulations of the wave.  "expect" holds the rule's picks, worked out by hand (in float64,
# with the margins stated); "pins" names the misreadings of ref_np.SELECT_VARIANTS the row is
# built against.  All rows: VL = 3, model sparse (one row per lane).

def _pin(kind, pins, expect, N0, N, W, P, c=1.0, m=1):
    k = len(N)
    return {"kind": kind, "model": "sparse", "k": k, "m": m, "c": float(F32(c)), "vl": 3.0,
            "N0": int(N0), "N": list(N), "W": [float(F32(x)) for x in W],
            "P": [float(F32(x)) for x in P], "expect": list(expect), "pins": list(pins)}


# The operand-order row: with c = 1.4f, Np = 5 and P = 0.000731f, (c*P)*s and c*(P*s) round to
# neighbouring floats.  Child 1 has N = 1, W = 0 (its score is exactly u / 2); child 0 has P = 0
# and W set so that its score W / 4 equals the smaller of the two roundings (halved): the rule
# then picks child 1 strictly, the misreading ties and takes child 0.
_PIN_OP_P = 0.000731
_PIN_OP_NP = 5


def _op_order_row():
    c, P = F32(1.4), F32(_PIN_OP_P)
    s = F32(np.sqrt(F32(_PIN_OP_NP)))
    u_rule = F32(F32(c * P) * s)
    u_alt = F32(c * F32(P * s))
    lo = min(u_rule, u_alt)
    w0 = F32(lo * F32(2.0))  # W/(1+3) = lo/2 exactly
    expect = [1] if u_rule > u_alt else [0]
    return _pin("pin_op_order", ["c_times_ps"], expect, _PIN_OP_NP - 3, [1, 1], [w0, 0.0],
                [0.0, _PIN_OP_P], c=1.4)


def pinned_row_cases() -> list[dict]:
    """Hand-built rows, each against named misreadings (see the block comment above)."""
    return [
        # Q over N + VL: child 0 Q = 0.9/4 = 0.225, child 1 Q = 5/13 = 0.385 (P = 0) -> 1.
        # With Q = W/N: 0.9 against 0.5 -> 0 (margins 0.16 and 0.4).
        _pin("pin_q_vl", ["q_no_vl"], [1], 10, [1, 10], [0.9, 5.0], [0.0, 0.0]),
        # sqrt(Np), Np = 1 + 3 = 4, s = 2: child 0 U = 0.42*2/2 = 0.42, child 1 Q = 1.78/4 =
        # 0.445 -> 1 (margin 0.025).  With sqrt(Np + 1) = 2.236: U = 0.4696 -> 0 (margin 0.025).
        _pin("pin_sqrt", ["sqrt_np_plus1"], [1], 1, [1, 1], [0.0, 1.78], [0.42, 0.0]),
        # the arriving VL in Np: s = sqrt(1 + 3) = 2, child 0 U = 0.42 against child 1 Q =
        # 1.2/4 = 0.3 -> 0 (margin 0.12).  With Np = 1 (VL added after the pick): U = 0.21 -> 1.
        _pin("pin_np_arrival", ["np_without_arrival"], [0], 1, [1, 1], [0.0, 1.2], [0.42, 0.0]),
        # exploration over 1 + N: child 0 U = 0.5*2/2 = 0.5, child 1 Q = 4.2/7 = 0.6 -> 1
        # (margin 0.1).  Over N: U = 1.0 -> 0 (margin 0.4).
        _pin("pin_denominator", ["denominator_n"], [1], 1, [1, 4], [0.0, 4.2], [0.5, 0.0]),
        # first unvisited child: child 1 has N = 0 -> 1.  Scored with Q = 0 instead:
        # child 0 = 4/8 + 0.1*sqrt(23)/6 = 0.580 against 0.01*sqrt(23) = 0.048 -> 0.
        _pin("pin_unvisited", ["no_unvisited_rule"], [1], 20, [5, 0], [4.0, 0.0], [0.1, 0.01]),
        # exact ties: three identical children -> 0 (lowest index); >= takes 2.
        _pin("pin_ties", ["ties_highest"], [0], 9, [5, 5, 5], [1.25] * 3, [0.25] * 3),
        # the children's in-flight VL: two identical children, two simulations.  The first
        # takes 0 (tie, Np = 12); then Np = 15 and child 0 has N = 8: Q + U = 1.25/11 +
        # 0.5*sqrt(15)/9 = 0.329 against child 1's 1.25/8 + 0.5*sqrt(15)/6 = 0.479 -> 1.
        # Without child 0's VL the tie repeats -> 0.
        _pin("pin_children_vl", ["children_no_vl"], [0, 1], 9, [5, 5], [1.25] * 2, [0.5] * 2,
             m=2),
        _op_order_row(),
    ]


def crafted_expected_np(case: dict, variant: str | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Picks (child index or -1 per simulation) and N after the wave, from the numpy
    restatement (with a planted misreading of ref_np.SELECT_VARIANTS when variant is set)."""
    k = case["k"]
    t = ref_np.NpTree(k + 1, case["c"], case["vl"], variant=variant)
    t.expand(0, list(range(k)), [F32(x) for x in case["P"]])
    t.N[0] = case["N0"]
    t.N[1:k + 1] = case["N"]
    t.W[1:k + 1] = case["W"]
    picks = []
    for _ in range(case["m"]):
        path = t.select_path(100)
        picks.append(path[1] - 1 if len(path) > 1 else -1)
    return np.array(picks, np.int32), t.N[:k + 1].copy()


def crafted_expected_oracle(case: dict) -> tuple[np.ndarray, np.ndarray]:
    """The same from the C oracle, on the crafted state written into its arrays."""
    k, m = case["k"], case["m"]
    model = model_from_name(case["model"])
    orc = Oracle(model, 1, k + 1, m, 100)
    orc.set_params(case["c"], case["vl"], 0, 0, 1.0, 0.0)
    orc.set_roots(games.root_keys(1, 1))
    orc.reset_tree(0)
    orc.write("N", np.concatenate([[case["N0"]], case["N"]]).astype(np.int32))
    orc.write("W", np.concatenate([[0.0], case["W"]]).astype(F32))
    orc.write("P", np.concatenate([[1.0], case["P"]]).astype(F32))
    orc.write("parent", np.array([-1] + [0] * k, np.int32))
    orc.write("first", np.array([0] + [-1] * k, np.int32))
    orc.write("nchild", np.array([k] + [0] * k, np.int32))
    orc.write("action", np.array([-1] + list(range(k)), np.int32))
    orc.write("expanded", np.array([1] + [0] * k, np.uint8))
    orc.write("children", np.arange(1, k + 1, dtype=np.int32))
    orc.write("child_actions", np.arange(k, dtype=np.int32))
    orc.write("num_nodes", np.array([k + 1], np.int32))
    orc.write("num_edges", np.array([k], np.int32))
    orc.lib.orc_wave_select(orc.f, 0, m, 100)
    lw = orc.last_wave(0, m)
    picks = np.array([p[1] - 1 if len(p) > 1 else -1 for p in lw["paths"]], np.int32)
    return picks, orc.array("N", k + 1)


META_KEYS = ("kind", "model", "k", "m", "c", "vl", "N0", "expect", "pins")


def pack_crafted(cases: list[dict], picks: list[np.ndarray], n_after: list[np.ndarray]) -> dict:
    """Flatten the cases into arrays for an npz file (no object arrays)."""
    meta = [{key: c[key] for key in META_KEYS if key in c} for c in cases]
    koff = np.concatenate([[0], np.cumsum([c["k"] for c in cases])]).astype(np.int64)
    moff = np.concatenate([[0], np.cumsum([c["m"] for c in cases])]).astype(np.int64)
    noff = np.concatenate([[0], np.cumsum([c["k"] + 1 for c in cases])]).astype(np.int64)
    return {
        "meta": np.array(json.dumps(meta)),
        "koff": koff, "moff": moff, "noff": noff,
        "N": np.concatenate([c["N"] for c in cases]).astype(np.int32),
        "W": np.concatenate([c["W"] for c in cases]).astype(F32),
        "P": np.concatenate([c["P"] for c in cases]).astype(F32),
        "picks": np.concatenate(picks).astype(np.int32),
        "N_after": np.concatenate(n_after).astype(np.int32),
    }


def unpack_crafted(z) -> list[dict]:
    meta = json.loads(str(z["meta"]))
    out = []
    for i, c in enumerate(meta):
        a, b = int(z["koff"][i]), int(z["koff"][i + 1])
        ma, mb = int(z["moff"][i]), int(z["moff"][i + 1])
        na, nb = int(z["noff"][i]), int(z["noff"][i + 1])
        c = dict(c)
        c.update(N=z["N"][a:b], W=z["W"][a:b], P=z["P"][a:b], picks=z["picks"][ma:mb],
                 N_after=z["N_after"][na:nb])
        out.append(c)
    return out


# ---- small whole searches with replayed evaluator rows ----------------------------------

SEARCH_CASES = [
    {"name": "gomoku4_full", "model": "gomoku:4", "policy": "full", "sign": 0, "eps": 0.0,
     "vl": 3.0, "W": 8, "sims": 96, "seed": 11, "stones": 3},
    {"name": "gomoku5_pw_rootpos_noise", "model": "gomoku:5", "policy": "reference_pw", "sign": 1,
     "eps": 0.25, "vl": 3.0, "W": 8, "sims": 96, "seed": 12, "stones": 4},
    {"name": "go4_full_vl1", "model": "go:4", "policy": "full", "sign": 0, "eps": 0.0,
     "vl": 1.0, "W": 5, "sims": 60, "seed": 13, "stones": 2},
    {"name": "gomoku4_vl0_ties", "model": "gomoku:4", "policy": "full", "sign": 0, "eps": 0.0,
     "vl": 0.0, "W": 3, "sims": 45, "seed": 14, "stones": 0},
]
CAPACITY = 4000
C_PUCT = 1.4


def search_inputs(case: dict) -> dict:
    """Root board, legal mask, keys, noise and the evaluator rows of every wave (seeded)."""
    model = model_from_name(case["model"])
    A, cells = model.num_actions, model.cells
    rng = np.random.default_rng(case["seed"])
    board = np.zeros(cells, np.int8)
    s = case["stones"]
    board[rng.permutation(cells)[:s]] = np.where(np.arange(s) % 2 == 0, 1, 2)
    legal = games.legal_masks(model, board.reshape(1, model.board_size, model.board_size), 1)
    root_legal = [a for a in range(A) if (int(legal[0, a // 32]) >> (a % 32)) & 1]
    noise = None
    if case["eps"] > 0:
        noise = np.zeros((1, A))
        noise[0, :len(root_legal)] = rng.dirichlet([0.3] * len(root_legal))
    W = case["W"]
    waves = [1] + [W] * (case["sims"] // W)
    pols, vals = [], []
    for wi in range(len(waves)):
        pol = rng.random((W, A)).astype(F32) + F32(0.01)
        val = (rng.random(W) * 2 - 1).astype(F32)
        if wi % 5 == 3:  # a wave of identical priors and values: exact ties
            pol[:] = F32(0.5)
            val[:] = F32(0.25)
        pols.append(pol)
        vals.append(val)
    return {"model": model, "board": board, "legal": legal, "root_legal": root_legal,
            "keys": games.root_keys(case["seed"], 1), "noise": noise, "waves": waves,
            "policy": np.stack(pols), "values": np.stack(vals)}


def search_expected(case: dict) -> dict:
    """Run the case on the C oracle and on the numpy restatement; both must agree.  Returns
    the per-wave paths (flattened) and the final tree."""
    inp = search_inputs(case)
    model = inp["model"]
    pass_action = model.num_actions - 1 if model.kind == "go" else None
    orc = Oracle(model, 1, CAPACITY, case["W"], 100)
    orc.set_params(C_PUCT, case["vl"], 1 if case["policy"] == "reference_pw" else 0, case["sign"],
                   1.0, case["eps"])
    orc.set_roots(inp["keys"], inp["legal"], inp["noise"])
    orc.reset_tree(0)
    npt = ref_np.NpTree(CAPACITY, C_PUCT, case["vl"])
    legal_of = lambda pacts: ref_np.board_legal(inp["root_legal"], pacts, pass_action)  # noqa: E731
    plens, pflat = [], []
    for wi, w in enumerate(inp["waves"]):
        pol, val = inp["policy"][wi], inp["values"][wi]
        orc.wave(0, w, replay_policy=pol, replay_values=val)
        paths, _ = ref_np.np_wave(npt, w, 100, legal_of, pol, val, case["policy"],
                                  None if inp["noise"] is None else inp["noise"][0], case["eps"],
                                  case["sign"] == 1)
        lw = orc.last_wave(0, w)
        for s in range(w):
            if list(lw["paths"][s]) != paths[s]:
                raise AssertionError(f"{case['name']} wave {wi} sim {s}: oracle "
                                     f"{list(lw['paths'][s])} numpy {paths[s]}")
            plens.append(len(paths[s]))
            pflat.extend(paths[s])
    tr = orc.tree(0)
    n = tr["num_nodes"]
    if n != npt.num_nodes:
        raise AssertionError(f"{case['name']}: node count {n} vs {npt.num_nodes}")
    for key in ("N", "parent", "first", "nchild", "action"):
        if not np.array_equal(tr[key], getattr(npt, key)[:n]):
            raise AssertionError(f"{case['name']}: {key} differs")
    for key in ("W", "P"):
        if not np.array_equal(tr[key].view(np.int32), getattr(npt, key)[:n].view(np.int32)):
            raise AssertionError(f"{case['name']}: {key} differs")
    out = {key: tr[key] for key in ("N", "W", "P", "parent", "first", "nchild", "action")}
    out["path_len"] = np.array(plens, np.int32)
    out["paths"] = np.array(pflat, np.int32)
    return out


# ---- progressive widening of the reference driver ----------------------------------------
# optimized_wave_search.py:394-415 and MAX_CHILDREN = 8 (cython_tree_optimized.pyx:31,239).
# The closed form below is written with integer square roots: floor(10 * sqrt(N0)) =
# isqrt(100 * N0) exactly (10 * sqrt(N0) is an integer only for square N0, where both are exact,
# and is at least 1 / (20 sqrt(N0) + 1) away from an integer otherwise).
PW_MODEL = "gomoku:5"
PW_GRID_N0 = (0, 1, 2, 3, 4, 9, 10, 16, 17, 20, 30, 100, 1000)
PW_GRID_L = (1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 12, 14, 15, 16, 20, 25)


def pw_root_count(N0: int, L: int) -> tuple[int, int]:
    """(size of the chosen set, row length) of a root with N0 visits and L legal actions:
    mc = max(5, min(L, floor(10 sqrt(N0)) + 1, 15)); chosen = the top-mc priors when L > mc,
    else all L; the row is the first min(8, chosen) of them."""
    import math

    mc = max(5, min(L, math.isqrt(100 * N0) + 1, 15))
    chosen = mc if L > mc else L
    return chosen, min(8, chosen)


def pw_inputs(L: int, seed: int):
    """A 5x5 Gomoku root with exactly L empty cells (stones elsewhere), its legal mask and a
    policy row of distinct values over the 25 cells (so that the order by prior has no ties).
    Returns (model, board int8[1,5,5], legal uint32[1,words], legal action list, policy
    float32[25])."""
    model = model_from_name(PW_MODEL)
    A = model.num_actions
    rng = np.random.default_rng(seed)
    board = np.zeros(A, np.int8)
    filled = rng.permutation(A)[:A - L]
    board[filled] = np.where(np.arange(A - L) % 2 == 0, 1, 2)
    board = board.reshape(1, model.board_size, model.board_size)
    legal = games.legal_masks(model, board, 1)
    acts = [a for a in range(A) if board.reshape(-1)[a] == 0]
    pol = ((rng.permutation(A) + 1) / (A * (A + 1) / 2)).astype(F32)
    return model, board, legal, acts, pol


def pw_expected(legal_actions, pol, N0: int | None):
    """Children actions (ascending) of a leaf under the rule: the root (N0 given) by
    pw_root_count, a non-root leaf (N0 None) the top min(3, L) priors.  The order by prior is
    taken on the raw policy row (renormalising over the legal set keeps the order of distinct
    values)."""
    L = len(legal_actions)
    by_prior = sorted(legal_actions, key=lambda a: (-float(pol[a]), a))
    if N0 is None:
        return sorted(by_prior[:min(3, L)])
    chosen, k = pw_root_count(N0, L)
    return sorted(by_prior[:chosen])[:k]


def pw_oracle_root(N0: int, L: int, seed: int, vl: float = 3.0):
    """The C oracle's root row after one simulation at a root with N0 visits and L legal
    actions (reference_pw), and the row of the root's first child after a second simulation."""
    model, board, legal, acts, pol = pw_inputs(L, seed)
    orc = Oracle(model, 1, 128, 1, 100)
    orc.set_params(1.4, vl, 1, 0, 1.0, 0.0)
    orc.set_roots(games.root_keys(seed, 1), legal)
    orc.reset_tree(0)
    orc.write("N", np.array([N0], np.int32))
    rows = np.stack([pol])
    orc.wave(0, 1, replay_policy=rows, replay_values=np.zeros(1, F32))
    tr = orc.tree(0)
    root = [int(a) for a in tr["action"][tr["first"][0] + 1:tr["first"][0] + 1 + tr["nchild"][0]]]
    child = None
    if tr["nchild"][0] > 0:
        orc.wave(0, 1, replay_policy=rows, replay_values=np.zeros(1, F32))
        tr = orc.tree(0)
        c0 = tr["first"][0] + 1
        f, k = tr["first"][c0], tr["nchild"][c0]
        child = [int(a) for a in tr["action"][f + 1:f + 1 + k]] if k > 0 else []
    return root, child
