"""Wave-by-wave parity harness: HIP library (WaveEngine) against the C oracle.

TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py cpu_baseline).

After every wave of every tree it compares, bit for bit: each simulation's path, the unique
leaves in first-occurrence order, and the whole used tree (N, W, P, parent, CSR row offset,
row length, action, node count).  W is compared bit-exactly in the ordered accumulation mode
and to 1e-5 relative otherwise.
"""
from __future__ import annotations

import numpy as np

from .oracle import Oracle

EXPAND_CODES = {"full": 0, "reference_pw": 1}


class ParityError(AssertionError):
    pass


def go_root_info(wl, seed=0):
    """Go root inputs for the rules: the workload's boards (empty when it has none), a ko
    point on an empty point for every other tree (-1 for the rest) and 0 or 1 root passes."""
    boards = wl.boards()
    bs = wl.model.board_size
    if boards is None:
        boards = np.zeros((wl.num_trees, bs, bs), np.int8)
    rng = np.random.default_rng(1000 + seed)
    ko = np.full(wl.num_trees, -1, np.int32)
    for t in range(0, wl.num_trees, 2):
        empty = np.flatnonzero(boards[t].reshape(-1) == 0)
        ko[t] = int(rng.choice(empty))
    passes = (np.arange(wl.num_trees) % 3 == 1).astype(np.int32)
    return boards, passes, ko


def make_pair(wl, max_wave=None, w_mode=0, vl_atomic=False, device="cuda", sign_mode=0,
              rule=None, go_flags=None):
    """Engine and oracle for the workload; rule (0 freestyle, 1 renju) turns the Gomoku
    terminal check on for both, from the workload's root boards; go_flags (1 ko, 2 suicide)
    the Go rules, from go_root_info."""
    from omoknuni_quantum_amd.core.engine import SearchParams, WaveEngine
    from omoknuni_quantum_amd.synthetic.evaluator import SyntheticEvaluator

    MW = max_wave or wl.wave_size
    params = SearchParams(c_puct=wl.c_puct, virtual_loss=wl.virtual_loss, max_depth=wl.max_depth,
                          expand_policy=EXPAND_CODES[wl.expand_policy], w_mode=w_mode,
                          sign_mode=sign_mode,
                          vl_atomic=vl_atomic, dirichlet_epsilon=wl.dirichlet_epsilon)
    eng = WaveEngine(wl.model, wl.num_trees, wl.capacity, MW, wl.max_depth, device, params)
    keys, legal, noise = wl.root_inputs()
    eng.set_roots(keys, legal, noise)
    orc = Oracle(wl.model, wl.num_trees, wl.capacity, MW, wl.max_depth)
    orc.set_params(wl.c_puct, wl.virtual_loss, EXPAND_CODES[wl.expand_policy], sign_mode,
                   wl.logit_scale, wl.dirichlet_epsilon)
    orc.set_roots(keys, legal, noise)
    if rule is not None:
        boards = wl.boards()
        if boards is None:
            boards = np.zeros((wl.num_trees, wl.model.board_size, wl.model.board_size), np.int8)
        eng.set_gomoku_rules(boards, rule)
        orc.set_gomoku_rules(boards, rule)
    if go_flags is not None:
        boards, passes, ko = go_root_info(wl)
        eng.set_go_rules(boards, go_flags, root_passes=passes, root_ko=ko)
        orc.set_go_rules(boards, go_flags, root_passes=passes, root_ko=ko)
    return eng, orc, SyntheticEvaluator(wl.logit_scale)


def _cmp(name, a, b, ctx):
    a = np.asarray(a)
    b = np.asarray(b)
    if a.shape != b.shape:
        raise ParityError(f"{ctx}: {name} shape {a.shape} != oracle {b.shape}")
    if a.dtype.kind == "f":
        eq = a.view(np.int32 if a.dtype == np.float32 else np.int64) == \
            b.astype(a.dtype).view(np.int32 if a.dtype == np.float32 else np.int64)
    else:
        eq = a == b
    if not np.all(eq):
        i = int(np.flatnonzero(~eq.reshape(-1))[0])
        raise ParityError(f"{ctx}: {name} differs at {i}: gpu {a.reshape(-1)[i]!r} "
                          f"oracle {b.reshape(-1)[i]!r} ({int((~eq).sum())} mismatches)")


def compare_wave(eng, orc, W, ctx, w_exact=True):
    """Compare the last wave and the trees of all T trees."""
    T, MW, MD = eng.T, eng.MW, eng.MD
    plen_all = eng.path_len.view(T, MW)[:, :W].cpu().numpy()
    paths_all = eng.paths.view(T, MW, MD)[:, :W].cpu().numpy()
    ucount = eng.ucount.cpu().numpy()
    uleaf_all = eng.uleaf.view(T, MW).cpu().numpy()
    for t in range(T):
        c = f"{ctx} tree {t}"
        lw = orc.last_wave(t, W)
        _cmp("path_len", plen_all[t], lw["path_len"], c)
        for s in range(W):
            L = plen_all[t, s]
            if not np.array_equal(paths_all[t, s, :L], lw["paths"][s]):
                raise ParityError(f"{c}: path of simulation {s} differs: gpu "
                                  f"{paths_all[t, s, :L].tolist()} oracle {lw['paths'][s].tolist()}")
        if ucount[t] != lw["ucount"]:
            raise ParityError(f"{c}: unique leaves {ucount[t]} != oracle {lw['ucount']}")
        _cmp("uleaf", uleaf_all[t, :ucount[t]], lw["uleaf"], c)
        if eng.rule is not None or eng.go_flags is not None:
            _cmp("uterm", eng.uterm.view(T, MW)[t, :ucount[t]].cpu().numpy(), lw["uterm"], c)
            _cmp("ulegal", eng.ulegal.view(T, MW)[t, :ucount[t]].cpu().numpy(), lw["ulegal"], c)
        g = eng.host_tree(t)
        o = orc.tree(t)
        if g["num_nodes"] != o["num_nodes"]:
            raise ParityError(f"{c}: num_nodes {g['num_nodes']} != oracle {o['num_nodes']}")
        for k in ("N", "parent", "first", "nchild", "action", "P"):
            _cmp(k, g[k], o[k], c)
        if w_exact:
            _cmp("W", g["W"], o["W"], c)
        else:
            err = np.abs(g["W"].astype(np.float64) - o["W"]) / np.maximum(1.0, np.abs(o["W"]))
            if err.size and err.max() > 1e-5:
                i = int(err.argmax())
                raise ParityError(f"{c}: W rel err {err.max():.3g} at {i}")
        # implicit CSR columns of the device layout = explicit edges of the oracle
        n = o["num_nodes"]
        if n > 1 and not np.array_equal(o["children"], np.arange(1, n, dtype=np.int32)):
            raise ParityError(f"{c}: oracle edge array is not child[e] = e+1")


def run_parity(wl, check_every=1, w_mode=0, vl_atomic=False, device="cuda", log=None,
               sign_mode=0, rule=None, stats=None, go_flags=None):
    """Run the whole search on both sides; compare after every check_every-th wave and at
    the end.  Returns the number of waves compared.  With a Gomoku rule or the Go rules,
    stats (a dict) receives the number of terminal unique leaves met."""
    import torch

    eng, orc, ev = make_pair(wl, w_mode=w_mode, vl_atomic=vl_atomic, device=device,
                             sign_mode=sign_mode, rule=rule, go_flags=go_flags)
    T = wl.num_trees
    eng.reset()
    for t in range(T):
        orc.reset_tree(t)
    sizes = [1]
    done = 0
    while done < wl.num_simulations:
        w = min(wl.wave_size, wl.num_simulations - done)
        sizes.append(w)
        done += w
    compared = 0
    for i, W in enumerate(sizes):
        eng.run_wave(W, ev)
        for t in range(T):
            orc.wave(t, W)
        if stats is not None and (rule is not None or go_flags is not None):
            for t in range(T):
                stats["terminal"] = stats.get("terminal", 0) + int(
                    (orc.last_wave(t, W)["uterm"] != 0).sum())
        if i % check_every == 0 or i == len(sizes) - 1:
            torch.cuda.synchronize()
            compare_wave(eng, orc, W, f"{wl.name} wave {i} (W={W})", w_exact=(w_mode == 0))
            compared += 1
            if log:
                log(f"{wl.name}: wave {i}/{len(sizes) - 1} W={W} parity ok")
    eng.check_status()
    pol_g = eng.root_policies()
    for t in range(T):
        if not np.allclose(pol_g[t], orc.root_policy(t), rtol=0, atol=1e-12):
            raise ParityError(f"{wl.name} tree {t}: root policy differs")
    return compared
