"""Benchmark of the wave-MCTS tree operations on one MI355X.

A step is one full search of the workload: every tree is reset, its root expanded, and
num_simulations simulations are run in waves (select -> synthetic evaluator -> expand ->
backup).  Inputs are resident in HBM before the timed region.  The metric is tree-operation
simulations per second: simulations / time of the tree-operation kernels (select, leaf info,
expand, backup), measured with HIP events on the launch stream; the synthetic evaluator is
timed apart.  Prints one JSON line: the headline workload (C3, the largest single-GPU config)
at the top level, then every other workload of the benchmark under "configs", each with its
roofline, CPU baseline and full-size parity check.

    python bench.py [--steps K] [--warmup W] [--config C3] [--configs all|none|C1,C2,...]
                    [--cpu-baseline auto|skip]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

_ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, _ROOT)

METRIC = "tree-op simulations/sec (synthetic evaluator) + achieved HBM GB/s, 1 GPU"
HBM_PEAK_GBS = 8000.0
TREE_PHASES = ("select", "leaf_info", "expand_backup")


def algorithmic_bytes(st: dict, sims: int, wave: int) -> dict:
    """Compulsory HBM bytes of each tree-operation kernel family over the timed region,
    from the device counters (the stats slots OMQ_ST_* of omq_tree_ops.h):
      select    16 B per visited node (row header N, first, nchild + N write of the virtual
                loss) + 12 B per child of each row scanned (N, W, P; a row whose picks are all
                first-unvisited children is scanned up to its last pick, where the reference's
                scan stops) + 4 B per path entry (path output) + 8 B per simulation (leaf and
                path length)
      records   the unique leaves' keys and legal counts: 8 B per path entry below the root of
                each unique leaf's path (the entry and its node's action) + 20 B per unique
                leaf (first simulation, path length, key, legal count).  Formed at the end of
                select for waves of at most OMQ_SELECT_RECORDS_MAX_WAVE simulations (counted
                with select), else by leaf_info_kernel (the leaf_info phase, which also holds
                the rule kernels when a rule is on; those are not modelled)
      expand_backup  (one phase: omq_expand_backup runs the two side by side)
        expand  8 B per expanded leaf (row header) + 28 B per child written (N, W, P, parent,
                action, row offset, row length) + 4 B per prior gathered (= per child in the
                full policy)
        backup  16 B per visited node (N and W read and written) + 4 B per path entry
                (signed leaf value read) + 12 B per simulation (value, uid, length)
    """
    from omoknuni_quantum_amd import _lib

    G, K, PE = st["pathnodes"], st["rowsum"], st["pathentries"]
    records = 8 * (st["uleafpath"] - st["uleaves"]) + 20 * st["uleaves"]
    in_select = wave <= _lib.OMQ_SELECT_RECORDS_MAX_WAVE
    return {
        "select": 16 * G + 12 * K + 4 * PE + 8 * sims + (records if in_select else 0),
        "leaf_info": 0 if in_select else records,
        "expand_backup": 8 * st["expanded"] + 32 * st["newchild"] + 16 * G + 4 * PE + 12 * sims,
    }



KERNEL_OF_PHASE = {"select": "select_root_kernel", "leaf_info": "leaf_info_kernel",
                   "expand_backup": "write_backup_kernel"}
ALL_CONFIGS = ("C1", "C2", "C3", "C4", "C5")


def parse_configs(spec: str) -> list[str]:
    if spec == "all":
        return list(ALL_CONFIGS)
    if spec in ("", "none"):
        return []
    out = [s.strip() for s in spec.split(",") if s.strip()]
    for s in out:
        if s not in ALL_CONFIGS:
            raise SystemExit(f"unknown workload {s!r}: one of {', '.join(ALL_CONFIGS)}")
    return out


def measured_traffic(workload: str, phase: str, args):
    """HBM bytes per launch of the phase's main kernel from the committed rocprofv3 --pmc
    summary (profiles/hbm_traffic.json: FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the
    same counters of a plain copy of known size).  None when no profile covers this run's
    workload and modes."""
    path = os.path.join(_ROOT, "profiles", "hbm_traffic.json")
    if args.w_mode != "ordered" or args.vl_atomic or args.trees or not os.path.exists(path):
        return None, None
    with open(path) as fh:
        table = json.load(fh)
    e = table.get(f"{workload}/{KERNEL_OF_PHASE[phase]}")
    if not e:
        return None, None
    return int(e["bytes_per_dispatch"]), e["source"]


def _engine(wl, args, dev):
    import torch

    from omoknuni_quantum_amd import _lib
    from omoknuni_quantum_amd.core.engine import SearchParams, WaveEngine
    from omoknuni_quantum_amd.synthetic.evaluator import SyntheticEvaluator

    params = SearchParams(c_puct=wl.c_puct, virtual_loss=wl.virtual_loss, max_depth=wl.max_depth,
                          expand_policy=_lib.OMQ_EXPAND_FULL,
                          w_mode=_lib.OMQ_WACC_ATOMIC if args.w_mode == "atomic" else _lib.OMQ_WACC_ORDERED,
                          vl_atomic=args.vl_atomic, dirichlet_epsilon=wl.dirichlet_epsilon)
    eng = WaveEngine(wl.model, wl.num_trees, wl.capacity, wl.wave_size, wl.max_depth, dev, params)
    keys, legal, noise = wl.root_inputs()
    eng.set_roots(keys, legal, noise)
    if wl.evaluator == "resnet":
        from omoknuni_quantum_amd.synthetic.resnet_evaluator import ResNetEvaluator
        boards = torch.from_numpy(wl.boards()).to(dev)
        ev = ResNetEvaluator(eng, boards)
    else:
        ev = SyntheticEvaluator(wl.logit_scale)
    return eng, ev


def measure(name: str, args, steps: int, warmup: int, extras: bool) -> dict:
    """One workload: warm-up searches, then `steps` timed searches (tree operations timed by
    HIP events on the launch stream), the roofline of the dominant kernel, and (unless
    skipped) the CPU baseline with the full-size parity check against it."""
    import torch

    from omoknuni_quantum_amd.core.timing import PhaseTimer
    from omoknuni_quantum_amd.synthetic.workloads import get

    wl = get(name)
    if args.trees:
        wl = wl.scaled(num_trees=args.trees)
    dev = torch.device("cuda:0")
    eng, ev = _engine(wl, args, dev)
    if args.copy_probe_mib > 0 and extras:
        # one plain device copy of known size, outside the timed region: the reference point
        # that scales the HBM counters (FETCH_SIZE / WRITE_SIZE) of a --pmc profile of this run
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize(dev)
        del src, dst
    for _ in range(warmup):
        eng.search(wl.num_simulations, wl.wave_size, ev)
    torch.cuda.synchronize(dev)
    eng.stats.zero_()
    timer = PhaseTimer(dev)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.search(wl.num_simulations, wl.wave_size, ev, timer)
    torch.cuda.synchronize(dev)
    t1 = time.perf_counter()
    eng.check_status()
    tot = timer.totals_ms()
    st = eng.host_stats()
    sims = wl.num_trees * wl.num_simulations * steps
    tree_ms = sum(tot.get(p, 0.0) for p in TREE_PHASES)
    eval_ms = tot.get("eval", 0.0)
    value = sims / (tree_ms / 1e3)
    ab = algorithmic_bytes(st, st["sims"], wl.wave_size)
    phases = {}
    for p in TREE_PHASES:
        n = timer.counts.get(p, 0)
        ms = tot.get(p, 0.0)
        phases[p] = {"ms_total": round(ms, 4), "launches": n,
                     "us_per_launch": round(1e3 * ms / max(n, 1), 3),
                     "algorithmic_GBps": round(ab[p] / (ms / 1e3) / 1e9, 2) if ms > 0 else None}
    dominant = max(TREE_PHASES, key=lambda p: tot.get(p, 0.0))
    dn = timer.counts[dominant]
    d_bytes = ab[dominant] / dn
    d_s = tot[dominant] / 1e3 / dn
    achieved = d_bytes / d_s / 1e9
    traffic, traffic_src = measured_traffic(wl.name, dominant, args)
    roofline = {"bound": "hbm", "kernel": KERNEL_OF_PHASE[dominant], "achieved": round(achieved, 2),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5),
                "traffic": traffic, "algorithmic_bytes_per_launch": int(d_bytes),
                "us_per_launch": round(d_s * 1e6, 3)}
    if traffic_src:
        roofline["traffic_source"] = traffic_src
    if dominant == "select":
        roofline["serial_floor"] = serial_floor(st, wl.num_trees, dn, d_s * 1e6)
    whole_bytes = sum(ab.values())
    out = {
        "value": round(value, 1),
        "ms_per_step": round(1e3 * (t1 - t0) / steps, 3),
        "config": {"workload": wl.name, "trees": wl.num_trees,
                   "simulations_per_tree": wl.num_simulations, "wave": wl.wave_size,
                   "capacity": wl.capacity, "game": wl.model.kind,
                   "actions": wl.model.num_actions, "w_mode": args.w_mode,
                   "vl_atomic": bool(args.vl_atomic),
                   "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "tree_op_ms_per_step": round(tree_ms / steps, 4),
        "eval_ms_per_step": round(eval_ms / steps, 4),
        "end_to_end_sims_per_s": round(sims / (t1 - t0), 1),
        "tree_op_algorithmic_GBps": round(whole_bytes / (tree_ms / 1e3) / 1e9, 2),
        "phases": phases,
        "counters": st,
    }
    if wl.evaluator == "resnet":
        out["evaluator"] = (f"random-init ResNet {ev.net.blocks.__len__()} blocks x 128 channels, "
                            "18 planes, bf16 weights and activations, batch norm folded, "
                            "channels-last, one forward pass per wave over "
                            f"{wl.num_trees} trees x {wl.wave_size} slots = "
                            f"{wl.num_trees * wl.wave_size} positions")
        out["tree_op_share"] = round(tree_ms / (tree_ms + eval_ms), 4)
        out["end_to_end_gpu_sims_per_s"] = round(sims / ((tree_ms + eval_ms) / 1e3), 1)
    if extras and args.graph and wl.evaluator == "synthetic":
        out["graph"] = graph_replay(wl, eng, ev, args)
    if args.cpu_baseline != "skip":
        replay = None
        if wl.evaluator == "resnet":
            # one more search with the evaluator outputs recorded, replayed into the oracle
            ev.record = True
            eng.search(wl.num_simulations, wl.wave_size, ev)
            torch.cuda.synchronize(dev)
            replay = ev.calls
        out["cpu_baseline"], out["parity_full_size"] = cpu_baseline(wl, eng, args, replay)
    if extras and args.next_rows != "skip":
        out["next_rows"] = next_rows(wl, eng, ev)
    del eng, ev
    torch.cuda.empty_cache()
    return out


def serial_floor(st, trees, launches, select_us) -> dict:
    """The selection's serial part: each tree's root chain (one dependent argmax step per
    simulation of the wave) runs before any deeper level can finish, so a launch takes at least
    its longest root chain.  The kernel times the chain with the device's constant wall clock
    (counter rootchain, ticks summed over trees and launches); the floor is its mean per tree
    and launch, beside the steps per launch, the time per step and select's time over it."""
    from omoknuni_quantum_amd import _lib

    khz = ctypes.c_int32(0)
    _lib.check(_lib.load().omq_wall_clock_khz(ctypes.byref(khz)), "omq_wall_clock_khz")
    chain_us = st["rootchain"] / (khz.value * 1e-3) / (trees * launches)
    steps = st["sims"] / (trees * launches)
    return {"root_chain_us_per_launch": round(chain_us, 3),
            "root_chain_steps_per_launch": round(steps, 1),
            "ns_per_step": round(1e3 * chain_us / steps, 2) if steps else None,
            "select_over_floor": round(select_us / chain_us, 3) if chain_us else None,
            "clock_khz": khz.value,
            "source": "counter rootchain (s_memrealtime around the root group's chain in "
                      "select_root_kernel), mean over the timed launches and trees"}


def run(args) -> dict:
    from omoknuni_quantum_amd import _lib

    _lib.check(_lib.load().omq_select_options(_lib.OMQ_SPIN_LIMIT_DEFAULT),
               "omq_select_options")
    head = measure(args.config, args, args.steps, args.warmup, extras=True)
    out = {
        "metric": METRIC,
        "value": head.pop("value"),
        "unit": "simulations/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
    }
    out.update(head)
    others = [c for c in parse_configs(args.configs) if c != args.config]
    if others:
        table = {}
        for name in others:
            e = measure(name, args, args.steps, min(args.warmup, 2), extras=False)
            e.pop("counters", None)
            table[name] = e
        out["configs"] = table
    return out


def graph_replay(wl, eng, ev, args) -> dict:
    """The whole search recorded once as a HIP graph and replayed: end-to-end time per search
    (tree operations and the synthetic evaluator), beside the eager end-to-end time."""
    import torch

    g = eng.capture_search(wl.num_simulations, wl.wave_size, ev)
    for _ in range(args.warmup):
        g.replay()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        g.replay()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    return {"ms_per_search": round(ms, 4),
            "end_to_end_sims_per_s": round(wl.num_trees * wl.num_simulations / (ms / 1e3), 1),
            "what": "select, leaf info, synthetic evaluator, expand and backup of every wave "
                    "of one search, replayed from one HIP graph"}


def next_rows(wl, eng, ev) -> dict:
    """The operations beside the wave path, timed once on the searched trees (after the
    parity check, outside the timed region): the Gomoku terminal check and the feature planes
    of one wave's leaves, the per-move root operations and the subtree reuse of every tree."""
    import torch

    from omoknuni_quantum_amd import _lib

    out = {}
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if wl.model.kind == "gomoku":
        # one more wave selected and its leaves looked up; the terminal check is then timed
        # alone over those leaves (repeated calls give the same result)
        boards = wl.boards()
        if boards is None:
            boards = np.zeros((wl.num_trees, wl.model.board_size, wl.model.board_size), np.int8)
        eng.set_gomoku_rules(boards, _lib.OMQ_RULE_FREESTYLE)
        eng.select(wl.wave_size)
        eng.leaf_info(wl.wave_size)
        reps = 20
        torch.cuda.synchronize()
        start.record()
        for _ in range(reps):
            eng.leaf_info_terminal_only()
        stop.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(stop) * 1e3 / reps
        nu = int(eng.ucount.sum().item())
        plen = eng.path_len.view(eng.T, eng.MW)
        first = eng.ufirst.view(eng.T, eng.MW).to(torch.int64).clamp_(0, eng.MW - 1)
        ucnt = eng.ucount.to(torch.int64)
        valid = torch.arange(eng.MW, device=eng.device)[None, :] < ucnt[:, None]
        moves = int(torch.where(valid, torch.gather(plen, 1, first) - 1, 0).sum().item())
        nterm = int((torch.where(valid, eng.uterm.view(eng.T, eng.MW), 0) != 0).sum().item())
        # per unique leaf: its root board (A bytes), 4 B per path move, 8 B written
        ab = nu * (wl.model.num_actions + 8) + 4 * moves
        out["gomoku_terminal"] = {
            "us_per_launch": round(us, 3), "unique_leaves": nu, "terminal_leaves": nterm,
            "algorithmic_bytes": ab, "algorithmic_GBps": round(ab / (us * 1e-6) / 1e9, 2),
            "launch": f"one wave of {wl.wave_size} simulations per tree after the timed "
                      f"searches, freestyle rule, {reps} launches averaged"}
        # feature planes of the same wave's slots: bfloat16 channels-last (the ResNet's input)
        # and float32 NCHW with the reference's 19 planes
        dev_boards = torch.from_numpy(boards.reshape(-1).copy()).to(eng.device)
        feats = {}
        for name, planes, dtype, nhwc in (("bf16_nhwc_18", 18, torch.bfloat16, True),
                                          ("f32_nchw_19", 19, torch.float32, False)):
            buf = torch.empty(eng.T * eng.MW * planes * eng.A, dtype=dtype, device=eng.device)
            eng.leaf_features(buf, dev_boards, planes, nhwc=nhwc)
            torch.cuda.synchronize()
            start.record()
            for _ in range(reps):
                eng.leaf_features(buf, dev_boards, planes, nhwc=nhwc)
            stop.record()
            torch.cuda.synchronize()
            us = start.elapsed_time(stop) * 1e3 / reps
            # every slot's planes written; per unique leaf its root board and path moves read
            ab = buf.numel() * buf.element_size() + nu * wl.model.num_actions + 4 * moves
            feats[name] = {"us_per_launch": round(us, 3), "algorithmic_bytes": ab,
                           "algorithmic_GBps": round(ab / (us * 1e-6) / 1e9, 2)}
        out["leaf_features"] = dict(feats, slots=eng.T * eng.MW, unique_leaves=nu,
                                    launch=f"the same wave's slots, {reps} launches averaged")
        eng.set_gomoku_rules(None)
    # per-move root operations: policy rows, a move per tree at temperature 1, root noise
    def timed(fn, reps=20):
        fn()
        torch.cuda.synchronize()
        start.record()
        for _ in range(reps):
            fn()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) * 1e3 / reps

    pol = eng.root_policies(device=True)
    acts = torch.empty(eng.T, dtype=torch.int32, device=eng.device)
    us_pol = timed(lambda: eng.lib.omq_root_policy(eng.forest_ref, pol.data_ptr(),
                                                    eng.stream_handle()))
    us_smp = timed(lambda: eng.lib.omq_sample_actions(eng.forest_ref, pol.data_ptr(), 1.0, 5, 1,
                                                       acts.data_ptr(), eng.stream_handle()))
    us_dir = timed(lambda: eng.lib.omq_root_dirichlet(eng.forest_ref, 0.3, 5, 1,
                                                       eng.noise.data_ptr(), eng.stream_handle()))
    out["root_ops"] = {
        "root_policy_us": round(us_pol, 3), "sample_actions_us": round(us_smp, 3),
        "root_dirichlet_us": round(us_dir, 3), "trees": eng.T, "actions": eng.A,
        "what": "one launch each over every tree (policy rows, one move per tree at "
                "temperature 1, Dirichlet(0.3) root noise), 20 launches averaged"}
    # subtree reuse: every tree moves to its most visited root child
    T, cap = eng.T, eng.cap
    roots = torch.arange(T, device=eng.device, dtype=torch.int64) * cap
    first = eng.first[roots].to(torch.int64)
    k = eng.nchild[roots].to(torch.int64)
    new_roots = np.full(T, -1, np.int32)
    kmax = int(k.max().item())
    if kmax > 0:
        j = torch.arange(kmax, device=eng.device)
        idx = roots[:, None] + first[:, None] + 1 + j[None, :]
        valid = j[None, :] < k[:, None]
        n = torch.where(valid, eng.N[torch.where(valid, idx, roots[:, None])], -1)
        best = n.argmax(dim=1)
        new_roots = (first + 1 + best).to(torch.int32).cpu().numpy()
        new_roots[(k == 0).cpu().numpy()] = -1
    before = int(eng.num_nodes.sum().item())
    eng.shift_roots(np.zeros(T, np.int32))  # workspace allocated outside the timed launch
    torch.cuda.synchronize()
    start.record()
    eng.shift_roots(new_roots)
    stop.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(stop) * 1e3
    kept = int(eng.num_nodes.sum().item())
    # per kept node: 24 B read (row, N, W, P, action) + 28 B written (the compacted record)
    ab = 52 * kept
    out["shift_root"] = {
        "us_per_launch": round(us, 3), "nodes_before": before, "nodes_kept": kept,
        "algorithmic_bytes": ab, "algorithmic_GBps": round(ab / (us * 1e-6) / 1e9, 2),
        "launch": "one launch, every tree moves to its most visited root child"}
    return out


# Host threads of the CPU baseline: one tree per thread, at most the CPU share of one GPU on
# the benchmark boxes (16 cores per GPU), whatever nproc reports there.
CPU_SHARE = 16


def _cpu_threads(T: int, args) -> tuple[int, int]:
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    want = args.cpu_threads or min(CPU_SHARE, avail)
    return max(1, min(want, T)), avail


def cpu_baseline(wl, eng, args, replay=None):
    """The C oracle (the CPU restatement of the reference tree path, gcc -O3) timed on the host
    on the same workload: the median of 5 searches after one warm-up, one tree per thread; and
    one thread on a bounded sample.  Its final trees are then compared bit for bit with the
    GPU's (the state after the last timed search: both searched the same roots)."""
    from oracle.oracle import Oracle
    from oracle.parity import EXPAND_CODES

    T = wl.num_trees if args.cpu_trees <= 0 else min(args.cpu_trees, wl.num_trees)
    keys, legal, noise = wl.root_inputs()
    orc = Oracle(wl.model, T, wl.capacity, wl.wave_size, wl.max_depth)
    orc.set_params(wl.c_puct, wl.virtual_loss, EXPAND_CODES[wl.expand_policy], 0, wl.logit_scale,
                   wl.dirichlet_epsilon)
    orc.set_roots(keys[:T], None if legal is None else legal[:T],
                  None if noise is None else noise[:T])
    reps = 5
    if replay is not None:
        # evaluator outputs recorded on the GPU, replayed wave by wave (one thread)
        sizes = [1]
        done = 0
        while done < wl.num_simulations:
            sizes.append(min(wl.wave_size, wl.num_simulations - done))
            done += sizes[-1]
        assert len(sizes) == len(replay)
        times = []
        for _ in range(1 + reps):
            t0 = time.perf_counter()
            for t in range(T):
                orc.reset_tree(t)
                for (pol, val), W in zip(replay, sizes):
                    orc.wave(t, W, replay_policy=pol[t], replay_values=val[t])
            times.append(time.perf_counter() - t0)
        dt = float(np.median(times[1:]))
        cpu = {"value": round(T * wl.num_simulations / dt, 1), "unit": "simulations/s",
               "cores": 1, "kind": "port",
               "sample": f"{T} of {wl.num_trees} trees x {wl.num_simulations} simulations of "
                         f"{wl.name}, tree operations only with the GPU run's evaluator outputs "
                         f"replayed; median of {reps} after 1 warm-up ({dt:.3f} s per search, "
                         "C oracle, gcc -O3, one thread)"}
    else:
        threads, avail = _cpu_threads(T, args)
        times = []
        for _ in range(1 + reps):
            t0 = time.perf_counter()
            orc.search(wl.num_simulations, wl.wave_size, wl.max_depth, nthreads=threads)
            times.append(time.perf_counter() - t0)
        dt = float(np.median(times[1:]))
        # single thread: whole trees, about 2 s of work at most
        t0 = time.perf_counter()
        t1 = 0
        while t1 < T and (t1 == 0 or time.perf_counter() - t0 < 2.0):
            orc.lib.orc_search_tree(orc.f, t1, wl.num_simulations, wl.wave_size, wl.max_depth)
            t1 += 1
        dt1 = time.perf_counter() - t0
        single = t1 * wl.num_simulations / dt1
        # (each search resets its trees: the last one leaves every tree as one full search)
        cpu = {"value": round(T * wl.num_simulations / dt, 1), "unit": "simulations/s",
               "cores": threads, "kind": "port",
               "sample": f"{T} of {wl.num_trees} trees x {wl.num_simulations} simulations of "
                         f"{wl.name}, one tree per thread on {threads} threads (the CPU share of "
                         f"one GPU on this box; {avail} cores visible), median of {reps} "
                         f"searches after 1 warm-up ({dt:.3f} s per search; C oracle, gcc -O3); "
                         f"single thread: {single:.1f} sims/s over {t1} tree(s) ({dt1:.2f} s)",
               "single_thread_value": round(single, 1), "host_cores_visible": avail}
    ok = True
    mismatch = None
    w_exact = args.w_mode == "ordered"
    for t in range(T):
        g = eng.host_tree(t)
        o = orc.tree(t)
        same = g["num_nodes"] == o["num_nodes"]
        for k in ("N", "parent", "first", "nchild", "action", "P"):
            same = same and np.array_equal(g[k], o[k])
        if same and w_exact:
            same = np.array_equal(g["W"].view(np.int32), o["W"].view(np.int32))
        elif same:
            same = np.allclose(g["W"], o["W"], rtol=1e-5, atol=1e-5)
        if not same:
            ok = False
            mismatch = t
            break
    parity = {"trees_compared": T, "bit_exact": ok, "first_mismatch_tree": mismatch,
              "compared": "N, W, P, parent, row offset, row length, action of every node"}
    return cpu, parity


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="C3",
                    help="the headline workload (the largest single-GPU config, C3, by default)")
    ap.add_argument("--configs", default="all",
                    help="workloads measured after the headline, in the same run: all, none, or "
                         "a comma-separated list of C1..C5")
    ap.add_argument("--trees", type=int, default=0, help="override the workload's tree count")
    ap.add_argument("--w-mode", choices=("ordered", "atomic"), default="ordered")
    ap.add_argument("--vl-atomic", action="store_true")
    ap.add_argument("--cpu-baseline", choices=("auto", "skip"), default="auto")
    ap.add_argument("--cpu-trees", type=int, default=0,
                    help="trees of the CPU baseline sample (0 = all)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="threads of the CPU baseline (0 = min(16, visible cores, trees))")
    ap.add_argument("--graph", action="store_true",
                    help="also time the search replayed from one HIP graph")
    ap.add_argument("--next-rows", choices=("auto", "skip"), default="auto",
                    help="also time the Gomoku terminal check and the subtree reuse once")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run one plain device copy of this size before the search (counter "
                         "calibration for --pmc profiles)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: the trees of a workload are "
                                   "independent and would be sharded one group per GPU; only "
                                   "--gpus 1 is measured"}))
        sys.exit(2)
    out = run(args)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
