"""Alternate modes of the wave operations and the reference-style primitives on the GPU."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd import _lib
from omoknuni_quantum_amd.core.engine import SearchParams, WaveEngine
from omoknuni_quantum_amd.synthetic import games
from omoknuni_quantum_amd.synthetic.evaluator import SyntheticEvaluator
from omoknuni_quantum_amd.synthetic.workloads import get
from oracle.parity import make_pair, run_parity

pytestmark = pytest.mark.gpu


def test_root_positive_sign_parity(device):
    wl = get("C1").scaled(name="C1-root_positive", num_simulations=480)
    assert run_parity(wl, sign_mode=_lib.OMQ_SIGN_ROOT_POSITIVE, device=device) >= 2


def test_atomic_virtual_loss_parity(device):
    wl = get("C2").scaled(name="C2-vl_atomic", num_trees=2, num_simulations=512, wave_size=256,
                          capacity=100_000)
    assert run_parity(wl, vl_atomic=True, device=device) >= 2


def test_atomic_w_within_tolerance(device):
    """W accumulated with float atomics stays within 1e-5 relative of the ordered sum, wave by
    wave; N is exact.  After each comparison the ordered W is copied over so the next selection
    starts from the same tree."""
    wl = get("C2").scaled(name="C2-atomic", num_trees=2, num_simulations=768, wave_size=256,
                          capacity=100_000)
    a, _, ev = make_pair(wl, w_mode=_lib.OMQ_WACC_ORDERED, device=device)
    b, _, _ = make_pair(wl, w_mode=_lib.OMQ_WACC_ATOMIC, device=device)
    a.reset()
    b.reset()
    for W in [1] + [256] * 3:
        a.run_wave(W, ev)
        b.run_wave(W, ev)
        torch.cuda.synchronize()
        assert torch.equal(a.N, b.N) and torch.equal(a.num_nodes, b.num_nodes)
        assert torch.equal(a.P, b.P)
        wa, wb = a.W.double(), b.W.double()
        rel = ((wa - wb).abs() / wa.abs().clamp_min(1.0)).max().item()
        assert rel <= 1e-5, rel
        b.W.copy_(a.W)


def _engine(T, cap, sign_mode=0, vl=3.0):
    params = SearchParams(virtual_loss=vl, sign_mode=sign_mode)
    return WaveEngine(games.gomoku(5), T, cap, 8, 16, "cuda", params)


@pytest.mark.parametrize("sign_mode", [0, 1])
def test_paths_backup_matches_numpy(device, sign_mode):
    T, cap, B, D = 3, 1000, 500, 12
    rng = np.random.default_rng(5 + sign_mode)
    eng = _engine(T, cap, sign_mode)
    paths = rng.integers(0, cap, (B, D)).astype(np.int32)
    plen = rng.integers(0, D + 1, B).astype(np.int32)
    for b in range(B):
        paths[b, plen[b]:] = -1
    paths[7, 2] = cap + 40          # out of range: skipped, the path goes on
    plen[7] = max(plen[7], 5)
    paths[7, :2] = [3, 4]
    paths[7, 3:plen[7]] = 9
    tree_of = rng.integers(0, T, B).astype(np.int32)
    tree_of[11] = T + 2             # names no tree: skipped
    values = (rng.integers(-8, 9, B) / 8.0).astype(np.float32)  # sums stay exact
    N = np.zeros((T, cap), np.int64)
    Wx = np.zeros((T, cap), np.float64)
    for b in range(B):
        t = tree_of[b]
        if t >= T:
            continue
        L = plen[b]
        for d in range(L):
            x = paths[b, d]
            if x < 0 or x >= cap:
                continue
            e = (L - 1 - d) if sign_mode == 0 else d
            N[t, x] += 1
            Wx[t, x] += -values[b] if e & 1 else values[b]
    eng.backup_paths(paths, plen, values, tree_of)
    torch.cuda.synchronize()
    assert np.array_equal(eng.N.view(T, cap).cpu().numpy(), N)
    assert np.array_equal(eng.W.view(T, cap).cpu().numpy().astype(np.float64), Wx)
    with pytest.raises(ValueError):
        eng.backup_paths(paths[:, 0], plen, values)


def test_virtual_loss_apply_revert(device):
    T, cap = 2, 64
    eng = _engine(T, cap, vl=3.0)
    eng.reset()
    base = eng.N.clone()
    nodes = np.array([0, 5, 5, 5, 63, -1, 64, 7], np.int32)
    tree_of = np.array([0, 1, 1, 0, 1, 0, 0, 9], np.int32)
    eng.apply_virtual_loss(nodes, tree_of)
    torch.cuda.synchronize()
    want = base.view(T, cap).cpu().numpy().copy()
    want[0, 0] += 3
    want[1, 5] += 6
    want[0, 5] += 3
    want[1, 63] += 3
    assert np.array_equal(eng.N.view(T, cap).cpu().numpy(), want)
    eng.remove_virtual_loss(nodes, tree_of)
    torch.cuda.synchronize()
    assert torch.equal(eng.N, base)
    eng.apply_virtual_loss([1, 2], amount=1)  # tree 0 when tree_of is omitted
    torch.cuda.synchronize()
    assert int(eng.N[1].item()) == int(base[1].item()) + 1


@pytest.mark.parametrize("name", ["C3", "C4"])
def test_synthetic_evaluator_rows_match_oracle(device, name):
    """Leaf keys, legal counts and values of the synthetic evaluator equal the oracle's."""
    wl = get(name).scaled(num_trees=2, num_simulations=128, wave_size=128, capacity=50_000)
    eng, orc, ev = make_pair(wl, device=device)
    eng.reset()
    for t in range(wl.num_trees):
        orc.reset_tree(t)
    for W in (1, 128):
        eng.run_wave(W, ev)
        for t in range(wl.num_trees):
            orc.wave(t, W)
    torch.cuda.synchronize()
    MW = eng.MW
    for t in range(wl.num_trees):
        lw = orc.last_wave(t, 128)
        u = lw["ucount"]
        assert int(eng.ucount[t].item()) == u
        keys = eng.ukey[t * MW:t * MW + u].cpu().numpy().view(np.uint64)
        assert np.array_equal(keys, lw["ukey"])
        assert np.array_equal(eng.ulegal[t * MW:t * MW + u].cpu().numpy(), lw["ulegal"])
        vals = eng.values[t * MW:t * MW + u].cpu().numpy()
        assert np.array_equal(vals.view(np.int32), lw["values"].view(np.int32))


def test_torch_ops_match_reference_kernel_semantics(device):
    """torch.ops.omq.* with the reference operator signatures (torch_custom_ops.py:26-55,
    mcts_kernels.cu:121-158,845-860,934-953)."""
    from omoknuni_quantum_amd import torch_ops  # noqa: F401  (registers the operators)

    rng = np.random.default_rng(3)
    n, B, D = 300, 200, 9
    paths = rng.integers(-1, n + 5, (B, D)).astype(np.int32)  # includes -1 and out-of-range
    plen = rng.integers(0, D + 4, B).astype(np.int32)  # lengths past the row: the sign still
    vals = (rng.integers(-16, 17, B) / 16.0).astype(np.float32)  # counts from the length given
    N = np.zeros(n, np.int64)
    Wx = np.zeros(n, np.float64)
    for b in range(B):
        for d in range(min(plen[b], D)):
            x = paths[b, d]
            if 0 <= x < n:
                N[x] += 1
                Wx[x] += vals[b] if (plen[b] - 1 - d) % 2 == 0 else -vals[b]
    vc = torch.zeros(n, dtype=torch.int32, device=device)
    vs = torch.zeros(n, dtype=torch.float32, device=device)
    torch.ops.omq.vectorized_backup(torch.from_numpy(paths).to(device),
                                    torch.from_numpy(plen).to(device),
                                    torch.from_numpy(vals).to(device), vc, vs)
    torch.cuda.synchronize()
    assert np.array_equal(vc.cpu().numpy(), N)
    assert np.array_equal(vs.cpu().numpy().astype(np.float64), Wx)
    idx = torch.tensor([1, 1, 2, -1, n + 3, 7], dtype=torch.int32, device=device)
    vl = torch.zeros(n, dtype=torch.int32, device=device)
    torch.ops.omq.batch_apply_virtual_loss(idx, vl)
    torch.cuda.synchronize()
    assert vl[1].item() == 2 and vl[2].item() == 1 and vl[7].item() == 1 and int(vl.sum()) == 4
    torch.ops.omq.batch_remove_virtual_loss(idx, vl)
    torch.cuda.synchronize()
    assert int(vl.abs().sum()) == 0


def test_count_limit_is_reported(device):
    """A root whose visit count plus the wave's virtual loss reaches 2^24 (forced from the
    host) sets OMQ_STATUS_COUNTLIMIT, and check_status raises; below it nothing is set."""
    wl = get("C2").scaled(num_trees=2, num_simulations=256, capacity=50_000)
    eng, orc, ev = make_pair(wl, device=device)
    eng.reset()
    eng.run_wave(1, ev)
    W = wl.wave_size
    vl = int(wl.virtual_loss)
    eng.N[0] = (1 << 24) - 1 - vl * W - 1  # tree 0: one below the limit
    eng.select(W)
    torch.cuda.synchronize()
    assert int(eng.status[0].item()) & _lib.OMQ_STATUS_COUNTLIMIT == 0
    eng.reset()
    eng.run_wave(1, ev)
    eng.N[eng.cap] = (1 << 24) - 1 - vl * W  # tree 1: at the limit
    eng.select(W)
    torch.cuda.synchronize()
    assert int(eng.status[0].item()) & _lib.OMQ_STATUS_COUNTLIMIT
    with pytest.raises(_lib.OmqError, match="2\\^24"):
        eng.check_status()
    eng.reset()
    eng.check_status()


def test_root_chain_counter_within_select_time(device):
    """The root-chain counter (OMQ_ST_ROOTCHAIN, wall-clock ticks) is positive after a search,
    and its mean per launch stays below select's own time per launch (the chain is part of the
    launch), which bench.py's serial floor relies on."""
    import ctypes
    from omoknuni_quantum_amd.core.timing import PhaseTimer

    wl = get("C3").scaled(name="C3-floor", num_trees=4, num_simulations=2048, capacity=800_000)
    params = SearchParams(c_puct=wl.c_puct, virtual_loss=wl.virtual_loss, max_depth=wl.max_depth,
                          dirichlet_epsilon=wl.dirichlet_epsilon)
    eng = WaveEngine(wl.model, wl.num_trees, wl.capacity, wl.wave_size, wl.max_depth, device,
                     params)
    eng.set_roots(*wl.root_inputs())
    ev = SyntheticEvaluator(wl.logit_scale)
    khz = ctypes.c_int32(0)
    _lib.check(_lib.load().omq_wall_clock_khz(ctypes.byref(khz)), "omq_wall_clock_khz")
    assert khz.value > 0
    eng.search(wl.num_simulations, wl.wave_size, ev)
    torch.cuda.synchronize()
    eng.stats.zero_()
    timer = PhaseTimer(torch.device(device))
    eng.search(wl.num_simulations, wl.wave_size, ev, timer)
    tot = timer.totals_ms()
    st = eng.host_stats()
    launches = timer.counts["select"]
    chain_ms = st["rootchain"] / khz.value / (wl.num_trees * launches)
    assert st["rootchain"] > 0
    assert 0.0 < chain_ms < tot["select"] / launches


@pytest.mark.gpu
@pytest.mark.parametrize("name,bs", [("C2", None), ("C4", None), ("C3", None), ("C3", 17),
                                     ("C2", 22)])
def test_select_leaf_records_equal_leaf_info(device, name, bs):
    """For a wave of at most OMQ_SELECT_RECORDS_MAX_WAVE simulations, omq_select forms the
    unique leaves' keys and legal counts itself; omq_leaf_info, run on the same wave, forms the
    same words (board and sparse models, select kernels of one, four, five, six and eight
    slots), so the two paths are interchangeable."""
    kw = {}
    if bs is not None:
        kw = {"model": games.go(bs) if name == "C3" else games.gomoku(bs), "max_stones": 40}
    wl = get(name).scaled(name=f"{name}-records", num_trees=3, num_simulations=1024,
                          wave_size=256, capacity=400_000, **kw)
    assert wl.wave_size <= _lib.OMQ_SELECT_RECORDS_MAX_WAVE
    params = SearchParams(c_puct=wl.c_puct, virtual_loss=wl.virtual_loss, max_depth=wl.max_depth,
                          dirichlet_epsilon=wl.dirichlet_epsilon)
    eng = WaveEngine(wl.model, wl.num_trees, wl.capacity, wl.wave_size, wl.max_depth, device,
                     params)
    eng.set_roots(*wl.root_inputs())
    ev = SyntheticEvaluator(wl.logit_scale)
    eng.search(3 * wl.wave_size, wl.wave_size, ev)  # a tree a few levels deep
    eng.select(wl.wave_size)
    torch.cuda.synchronize()
    T, MW = eng.T, eng.MW
    nu = eng.ucount.cpu().numpy()
    assert nu.min() > 0
    key_s = eng.ukey.view(T, MW).cpu().numpy()
    legal_s = eng.ulegal.view(T, MW).cpu().numpy()
    eng.ukey.fill_(0)
    eng.ulegal.fill_(-1)
    torch.cuda.synchronize()
    _lib.check(eng.lib.omq_leaf_info(eng.forest_ref, eng.wave_ref, eng.stream_handle()),
               "omq_leaf_info")
    torch.cuda.synchronize()
    key_i = eng.ukey.view(T, MW).cpu().numpy()
    legal_i = eng.ulegal.view(T, MW).cpu().numpy()
    for t in range(T):
        n = int(nu[t])
        assert (key_s[t, :n] == key_i[t, :n]).all()
        assert (legal_s[t, :n] == legal_i[t, :n]).all()
        assert (legal_s[t, :n] >= 0).all()


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw", [
    ("C2", {"num_trees": 3, "num_simulations": 1024, "wave_size": 256, "capacity": 200_000}),
    ("C3", {"num_trees": 2, "num_simulations": 3072, "wave_size": 1024, "capacity": 500_000}),
    ("C4", {"num_trees": 2, "num_simulations": 4096, "wave_size": 2048, "capacity": 200_000}),
])
def test_expand_backup_equals_expand_then_backup(device, name, kw):
    """omq_expand_backup (the expansion's and the backup's kernels side by side) leaves every
    node's N, W, P, parent, action and row exactly as omq_expand followed by omq_backup."""
    wl = get(name).scaled(name=f"{name}-expand-backup", **kw)
    params = SearchParams(c_puct=wl.c_puct, virtual_loss=wl.virtual_loss, max_depth=wl.max_depth,
                          dirichlet_epsilon=wl.dirichlet_epsilon)
    engs = []
    for _ in range(2):
        e = WaveEngine(wl.model, wl.num_trees, wl.capacity, wl.wave_size, wl.max_depth, device,
                       params)
        e.set_roots(*wl.root_inputs())
        e.reset()
        engs.append(e)
    ev = SyntheticEvaluator(wl.logit_scale)
    sizes = [1] + [wl.wave_size] * ((wl.num_simulations - 1) // wl.wave_size)
    for W in sizes:
        engs[0].run_wave(W, ev)  # omq_expand_backup
        e = engs[1]
        e.select(W)
        if e.needs_leaf_info(W):
            e.leaf_info(W)
        ev.evaluate_wave(e)
        e.expand(W)
        e.backup(W)
    torch.cuda.synchronize()
    for e in engs:
        e.check_status()
    a, b = engs
    assert torch.equal(a.num_nodes, b.num_nodes)
    for name_ in ("N", "W", "P", "parent", "first", "nchild", "action"):
        x, y = getattr(a, name_), getattr(b, name_)
        assert torch.equal(x.view(torch.int32) if x.dtype == torch.float32 else x,
                           y.view(torch.int32) if y.dtype == torch.float32 else y), name_
