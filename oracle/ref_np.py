"""Independent numpy-float32 restatement of the reference CPU tree semantics, for tiny trees.

TEST INFRASTRUCTURE ONLY (imported by tests/).  It pins the C oracle (oracle/tree_oracle.c):
both are written from the reference's behaviour, separately, and must agree bit for bit.

Reference behaviour restated (cosmosapjw-quantum/omoknuni_quantum):
  init .............. python/mcts/cpu/cython_tree_optimized.pyx:92-100 (N[0]=1, P[0]=1)
  best child ........ cython_tree_optimized.pyx:421-464
  select_path ....... cython_tree_optimized.pyx:177-202 (+VL on arrival)
  expand_node ....... cython_tree_optimized.pyx:232-277 (contiguous nodes and edges)
  backup ............ VL revert of cython_tree_optimized.pyx:222, sign of
                      python/mcts/cpu/optimized_wave_search.py:472-483 (leaf-positive) or
                      cython_tree_optimized.pyx:216-224 (root-positive)
  expansion policy .. optimized_wave_search.py:377-415 (legal renormalisation; 'full' or the
                      reference's progressive widening)
numpy float32 scalar arithmetic is IEEE binary32 with round-to-nearest-even, which is the
arithmetic the reference's Cython tree performs in source order.
"""
from __future__ import annotations

import math

import numpy as np

F = np.float32


def sum64(x) -> np.float32:
    """Canonical 64-lane sum: lane l adds elements l, l+64, ... from +0 in order, then the xor
    butterfly 32, 16, 8, 4, 2, 1."""
    part = [F(0.0)] * 64
    for i, v in enumerate(x):
        part[i % 64] = F(part[i % 64] + F(v))
    off = 32
    while off >= 1:
        part = [F(part[l] + part[l ^ off]) for l in range(64)]
        off //= 2
    return part[0]


def sum64d(x) -> float:
    part = [0.0] * 64
    for i, v in enumerate(x):
        part[i % 64] = part[i % 64] + float(v)
    off = 32
    while off >= 1:
        part = [part[l] + part[l ^ off] for l in range(64)]
        off //= 2
    return part[0]


# Planted misreadings of the selection rule (cython_tree_optimized.pyx:177-202,421-464), used
# only by the tests that show the pinning checks fail on each of them.  None is the rule.
SELECT_VARIANTS = (
    "q_no_vl",             # Q = W / N instead of W / (N + VL)
    "sqrt_np_plus1",       # sqrt(Np + 1) instead of sqrt(Np)
    "np_without_arrival",  # the arriving simulation's VL added to the parent after the pick
    "denominator_n",       # exploration over N instead of 1 + N
    "c_times_ps",          # c * (P * s) instead of (c * P) * s
    "no_unvisited_rule",   # unvisited children scored (Q = 0) instead of taken first
    "ties_highest",        # >= instead of > (ties to the highest index)
    "children_no_vl",      # children scored without the in-flight VL of earlier simulations
)


# Planted misreadings of the capacity rule of expand_node (cython_tree_optimized.pyx:242-246:
# a leaf whose n children do not fit is refused whole, and later leaves are still tried), used
# only by the tests that show the capacity checks fail on each of them.  None is the rule.
CAP_VARIANTS = (
    "first_fail",  # after the first refusal of a wave, every later leaf of it refused too
    "partial",     # a leaf that does not fit gets as many children as still fit
)


class NpTree:
    def __init__(self, cap: int, c_puct: float, vl: float, variant: str | None = None,
                 cap_variant: str | None = None):
        if variant is not None and variant not in SELECT_VARIANTS:
            raise ValueError(f"unknown selection variant {variant!r}")
        if cap_variant is not None and cap_variant not in CAP_VARIANTS:
            raise ValueError(f"unknown capacity variant {cap_variant!r}")
        self.variant = variant
        self.cap_variant = cap_variant
        self.wave_refused = False  # a refusal happened in the current wave (first_fail)
        self.inflight = np.zeros(cap, np.int32)  # simulations of the current wave per node
        self.cap = cap
        self.c = F(c_puct)
        self.vlf = F(vl)
        self.vli = int(vl)
        self.N = np.zeros(cap, np.int32)
        self.W = np.zeros(cap, np.float32)
        self.P = np.zeros(cap, np.float32)
        self.parent = np.full(cap, -1, np.int32)
        self.first = np.full(cap, -1, np.int32)
        self.nchild = np.zeros(cap, np.int32)
        self.action = np.zeros(cap, np.int32)
        self.expanded = np.zeros(cap, bool)
        self.children = np.zeros(cap, np.int32)
        self.num_nodes = 1
        self.num_edges = 0
        self.N[0] = 1
        self.P[0] = F(1.0)
        self.action[0] = -1

    def best_child(self, p: int, Np: int | None = None) -> int:
        Np = int(self.N[p]) if Np is None else Np
        f, k = int(self.first[p]), int(self.nchild[p])
        if k == 0 or f < 0 or Np == 0:
            return -1
        var = self.variant
        s = F(math.sqrt(float(F(Np + 1 if var == "sqrt_np_plus1" else Np))))
        best, arg = F(-1e9), -1
        for i in range(k):
            ch = int(self.children[f + i])
            n = int(self.N[ch])
            if var == "children_no_vl":
                n -= self.vli * int(self.inflight[ch])
            if n == 0 and var != "no_unvisited_rule":
                return ch
            if var == "q_no_vl":
                q = F(self.W[ch] / F(n)) if n > 0 else F(0.0)
            elif var == "no_unvisited_rule" and n == 0:
                q = F(0.0)
            else:
                q = F(self.W[ch] / F(F(n) + self.vlf))
            if var == "c_times_ps":
                num = F(self.c * F(self.P[ch] * s))
            else:
                num = F(F(self.c * self.P[ch]) * s)
            u = F(num / F(n if (var == "denominator_n" and n > 0) else 1 + n))
            sc = F(q + u)
            if sc > best or (var == "ties_highest" and sc == best):
                best, arg = sc, ch
        return arg

    def select_path(self, max_depth: int):
        path, cur = [], 0
        late = self.variant == "np_without_arrival"
        while True:
            path.append(cur)
            self.inflight[cur] += 1
            if not late:
                self.N[cur] += self.vli
            if not self.expanded[cur] or self.nchild[cur] == 0 or len(path) == max_depth:
                if late:
                    self.N[cur] += self.vli
                return path
            c = self.best_child(cur)
            if late:
                self.N[cur] += self.vli
            if c < 0:
                return path
            cur = c

    def expand(self, leaf: int, actions, priors) -> bool:
        k = len(actions)
        if self.expanded[leaf] or k == 0:
            return False
        if self.cap_variant == "first_fail" and self.wave_refused:
            return False
        if self.num_nodes + k > self.cap:
            if self.cap_variant == "partial" and self.num_nodes < self.cap:
                k = self.cap - self.num_nodes
            else:
                self.wave_refused = True
                return False
        fe, fc = self.num_edges, self.num_nodes
        self.num_edges += k
        self.num_nodes += k
        self.first[leaf], self.nchild[leaf], self.expanded[leaf] = fe, k, True
        for j in range(k):
            c = fc + j
            self.parent[c], self.P[c], self.action[c] = leaf, F(priors[j]), actions[j]
            self.N[c], self.W[c] = 0, F(0.0)
            self.children[fe + j] = c
        return True

    def shift_root(self, r: int) -> dict:
        """CSRTree.shift_root (python/mcts/gpu/csr_tree.py:1020-1229): breadth-first from r
        over each node's children (its row, in order), new index = discovery order; node
        data copied, parents remapped, the root's parent and action cleared; rows rebuilt
        node by node in the new order.  Returns the old -> new mapping."""
        if r == 0 or not (0 < r < self.num_nodes):
            return {i: i for i in range(self.num_nodes)}
        order, new_of = [r], {r: 0}
        head = 0
        while head < len(order):
            cur = order[head]
            head += 1
            f, k = int(self.first[cur]), int(self.nchild[cur])
            for ch in (self.children[f:f + k] if f >= 0 else []):
                ch = int(ch)
                if ch not in new_of:
                    new_of[ch] = len(order)
                    order.append(ch)
        old = {k: getattr(self, k)[order].copy() for k in ("N", "W", "P", "action", "expanded")}
        old_par = self.parent[order].copy()
        rows = [[new_of[int(c)] for c in (self.children[int(self.first[o]):int(self.first[o]) +
                                                          int(self.nchild[o])]
                                          if self.first[o] >= 0 else [])] for o in order]
        n = len(order)
        n_old = self.num_nodes
        # the reference resets the whole tree before writing the kept nodes back
        self.N[:n_old], self.W[:n_old], self.P[:n_old] = 0, F(0.0), F(0.0)
        self.parent[:n_old], self.first[:n_old], self.nchild[:n_old] = -1, -1, 0
        self.action[:n_old], self.expanded[:n_old], self.children[:n_old] = 0, False, 0
        for k, v in old.items():
            getattr(self, k)[:n] = v
        self.parent[:n] = [new_of.get(int(p), -1) if p >= 0 else -1 for p in old_par]
        self.parent[0] = -1
        self.action[0] = -1
        e = 0
        for i, row in enumerate(rows):
            self.first[i] = e if row else -1
            self.nchild[i] = len(row)
            for c in row:
                self.children[e] = c
                e += 1
        self.num_nodes, self.num_edges = n, e
        return new_of

    def backup(self, path, v: float, root_positive: bool = False):
        L = len(path)
        v = F(v)
        for d, x in enumerate(path):
            e = d if root_positive else L - 1 - d
            self.inflight[x] -= 1
            self.N[x] = self.N[x] - self.vli + 1
            self.W[x] = F(self.W[x] + (-v if e & 1 else v))


# Planted misreadings of the reference's progressive widening (optimized_wave_search.py:394-415
# and MAX_CHILDREN = 8 of cython_tree_optimized.pyx:31,239), used only by the tests that show
# the widening checks fail on each of them.  None is the rule.
PW_VARIANTS = (
    "no_plus1",      # int(10 * sqrt(N0)) without the + 1
    "no_floor5",     # without max(5, .)
    "no_cap15",      # without min(., 15)
    "no_cap8",       # the root row not cut to MAX_CHILDREN = 8
    "top8_by_prior", # the root's children: the 8 best priors instead of the 8 lowest actions
    "nonroot_top5",  # non-root rows of 5 instead of 3
)


# Planted misreadings of the root Dirichlet mix (optimized_wave_search.py:384-392 under numpy's
# promotion: float32 priors times the Python float 1 - eps stay float32, the float64 noise
# term promotes the sum to float64; cython_tree_optimized.pyx:569-572 rounds it to float32),
# used only by the tests that show the mix checks fail on each of them.  None is the rule.
MIX_VARIANTS = (
    "mix_f32",           # the whole mix in float32 (noise rounded to float32 first)
    "w_double",          # (1 - eps) * p formed in float64 instead of float32
    "renorm_double",     # the legal renormalisation p / S kept in float64 before the mix
    "mixed_rounded",     # the mixed prior rounded to float32 before the widening's renorm
    "renorm_after_mix",  # under 'full', the mixed priors renormalised by their sum
    "pw_renorm_f32",     # the widening's renormalisation of noisy priors in float32
)


def choose_children(legal, pol_row, is_root, policy, root_visits, noise=None, eps=0.0,
                    pw_variant=None, mix_variant=None):
    """Expansion of one leaf (optimized_wave_search.py:377-415): legal priors renormalised by
    their canonical sum, Dirichlet at the root, 'full' or progressive widening; returns
    (actions, priors) in ascending action order.  pw_variant plants a misreading of
    PW_VARIANTS, mix_variant one of MIX_VARIANTS."""
    if pw_variant is not None and pw_variant not in PW_VARIANTS:
        raise ValueError(f"unknown widening variant {pw_variant!r}")
    if mix_variant is not None and mix_variant not in MIX_VARIANTS:
        raise ValueError(f"unknown mix variant {mix_variant!r}")
    mv = mix_variant
    legal = list(legal)
    n = len(legal)
    pf = [F(pol_row[a]) for a in legal]
    S = sum64(pf)
    if mv == "renorm_double":
        pr = [float(p) / float(S) for p in pf]
    else:
        pr = [float(F(p / S)) for p in pf]
    pf = [F(p) for p in pr]
    noisy = is_root and noise is not None and eps > 0
    w32 = F(1.0 - eps)

    def mix(i):
        if mv == "mix_f32":
            return float(F(F(w32 * pf[i]) + F(F(eps) * F(noise[i]))))
        if mv == "w_double":
            return (1.0 - eps) * pr[i] + eps * float(noise[i])
        if mv == "renorm_double":
            return float(w32) * pr[i] + eps * float(noise[i])
        x = float(F(w32 * pf[i])) + eps * float(noise[i])
        return float(F(x)) if mv == "mixed_rounded" else x

    pd = [mix(i) if noisy else float(p) for i, p in enumerate(pf)]
    if noisy and mv == "renorm_after_mix" and policy == "full":
        Sm = sum64d(pd)
        pd = [x / Sm for x in pd]
    chosen = list(range(n))
    k = n
    if policy == "reference_pw":
        if is_root:
            plus = 0 if pw_variant == "no_plus1" else 1
            m1 = min(n, int(10.0 * math.sqrt(float(root_visits))) + plus)
            sel = m1 if pw_variant == "no_cap15" else min(m1, 15)
            sel = sel if pw_variant == "no_floor5" else max(5, sel)
        else:
            sel = 5 if pw_variant == "nonroot_top5" else 3
        if n > sel:
            order = sorted(range(n), key=lambda i: (-pd[i], i))[:sel]
            chosen = sorted(order)
            if noisy and mv != "pw_renorm_f32":
                Sd = sum64d([pd[i] for i in chosen])
                for i in chosen:
                    pd[i] = pd[i] / Sd
            else:
                Sf = sum64([F(pd[i]) for i in chosen])
                for i in chosen:
                    pd[i] = float(F(F(pd[i]) / Sf))
        k = min(len(chosen), 8) if is_root and pw_variant != "no_cap8" else len(chosen)
        if is_root and pw_variant == "top8_by_prior":
            chosen = sorted(sorted(chosen, key=lambda i: (-pd[i], i))[:k])
    chosen = chosen[:k]
    return [legal[i] for i in chosen], [F(pd[i]) for i in chosen]


def gomoku_terminal(board, renju: bool = False) -> int:
    """Full-board Gomoku scan of FastTerminalChecker._check_gomoku_terminal_cpu without a last
    move (python/mcts/utils/fast_terminal_check.py:132-232), on a [bs, bs] board of 0/1/2.

    All five-windows are found with array slices, per direction in the reference's order
    (horizontal, vertical, down-right, down-left).  The cells are then visited in row-major
    order.  At each occupied cell, the first direction whose window is full decides: an
    overline of player 1 under renju skips the cell, anything else returns the player.
    Returns 1 or 2 for a win, 3 for a full board without a five, 0 otherwise."""
    b = np.asarray(board, dtype=np.int64)
    bs = b.shape[0]
    dirs = ((0, 1), (1, 0), (1, 1), (1, -1))
    full = np.zeros((4, bs, bs), bool)
    over = np.zeros((4, bs, bs), bool)

    def at(r, c):
        return b[r, c] if 0 <= r < bs and 0 <= c < bs else -1

    for d, (dr, dc) in enumerate(dirs):
        for r in range(bs):
            for c in range(bs):
                re, ce = r + 4 * dr, c + 4 * dc
                if not (re < bs and 0 <= ce < bs) or b[r, c] == 0:
                    continue
                cells = [b[r + k * dr, c + k * dc] for k in range(5)]
                if all(x == b[r, c] for x in cells):
                    full[d, r, c] = True
                    over[d, r, c] = (at(r + 5 * dr, c + 5 * dc) == b[r, c]
                                     or at(r - dr, c - dc) == b[r, c])
    for r in range(bs):
        for c in range(bs):
            ds = np.flatnonzero(full[:, r, c])
            if len(ds) == 0:
                continue
            d = int(ds[0])
            if renju and b[r, c] == 1 and over[d, r, c]:
                continue
            return int(b[r, c])
    return 3 if np.all(b != 0) else 0


def leaf_position(root_board, path_actions, root_player=None, root_moves=None):
    """Position after the moves of a path, as CPUGameStates.apply_actions leaves it
    (python/mcts/cpu/cpu_game_states.py:372-384): each move puts the current player's stone on
    cell (a // bs, a % bs), switches the player and adds one to the move count.  The root's
    player and move count are those MCTS gives an ndarray root (python/mcts/core/mcts.py:
    1503-1508): player 1 when the stone count is even, else 2, and the stone count.
    Returns (board int8 [bs, bs], player to move, move count)."""
    b = np.array(root_board, dtype=np.int8, copy=True)
    bs = b.shape[0]
    stones = int(np.count_nonzero(b))
    player = (1 if stones % 2 == 0 else 2) if root_player is None else int(root_player)
    count = stones if root_moves is None else int(root_moves)
    for a in path_actions:
        b[a // bs, a % bs] = player
        player = 3 - player
        count += 1
    return b, player, count


def nn_features(board, player, move_count, planes: int = 19):
    """CPUGameStates.get_nn_features, representation 'basic' (python/mcts/cpu/
    cpu_game_states.py:452-494), of one position: float32 [planes, bs, bs] with
    0 the player's stones, 1 the opponent's, 2-15 zero, 16 ones when player 1 is to move,
    17 move_count / 100 (int16 count over a Python float: a double division, stored as
    float32), 18 ones.  planes=18 leaves out the last plane."""
    bs = board.shape[0]
    f = np.zeros((19, bs, bs), dtype=np.float32)
    f[0] = (board == player).astype(np.float32)
    f[1] = (board == 3 - player).astype(np.float32)
    f[16] = float(player == 1)
    f[17] = np.int16(move_count) / 100.0
    f[18] = 1.0
    return f[:planes]


# Planted misreadings of the Go rules, used only by the tests that show the known answers fail
# on each of them.  None is the rule.
GO_VARIANTS = (
    "ko_root_only",        # the ko point excluded at the root only (clones do inherit it)
    "suicide_diagonal",    # diagonal empty points counted as liberties
    "no_suicide_check",    # occupied neighbours counted as liberties too (no check at all)
    "passes_no_root",      # the root's own trailing passes not counted
    "passes_any_two",      # any two passes on the path, not two consecutive ones
    "full_not_terminal",   # a board without an empty point not terminal
    "pass_not_legal",      # the pass left out of the legal moves
    "root_terminal",       # the root itself checked for two passes
)


def go_rules(root_board, path_actions, root_player=None, root_passes=0, ko=-1, flags=1,
             variant=None):
    """Go rules of the position after the path moves: (legal moves ascending, terminal).

    * The position: the root board with the moves played alternately from the root's player
      (1 for an even stone count when not given), a pass (action bs*bs) placing no stone and no
      stone ever captured (GPUGameStates.apply_moves, python/mcts/gpu/gpu_game_states.py:
      430-441).
    * Legal: empty points; with flags & 1 not the root's ko point, which every descendant
      inherits (get_legal_moves_mask :373-395, clone_states :336-337); with flags & 2 only the
      points whose 4-neighbourhood holds an empty point (go_kernels.py:46-110, the liberty
      count of a 0/1 empty map convolved with the plus-shaped kernel, zero padding); then the
      pass.
    * Terminal (go_kernels.py:17-44), for a path of at least one move: the last two moves are
      passes (the root's trailing passes prepended), or no point is empty.

    Written with array operations (a padded empty map and shifted sums), independently of the
    C oracle's point loop."""
    b = np.array(root_board, dtype=np.int8, copy=True)
    bs = b.shape[0]
    cells = bs * bs
    stones = int(np.count_nonzero(b))
    player = (1 if stones % 2 == 0 else 2) if root_player is None else int(root_player)
    flat = b.reshape(-1)
    for a in path_actions:
        if a != cells:
            flat[a] = player
        player = 3 - player
    empty = (b == 0)
    legal = empty.copy()
    if flags & 1 and ko >= 0 and not (variant == "ko_root_only" and len(path_actions) > 0):
        legal.reshape(-1)[ko] = False
    if flags & 2:
        pad = np.zeros((bs + 2, bs + 2), np.int32)
        pad[1:-1, 1:-1] = empty
        libs = pad[:-2, 1:-1] + pad[2:, 1:-1] + pad[1:-1, :-2] + pad[1:-1, 2:]
        if variant == "suicide_diagonal":
            libs = libs + pad[:-2, :-2] + pad[:-2, 2:] + pad[2:, :-2] + pad[2:, 2:]
        if variant == "no_suicide_check":
            pad[1:-1, 1:-1] = 1
            libs = pad[:-2, 1:-1] + pad[2:, 1:-1] + pad[1:-1, :-2] + pad[1:-1, 2:]
        legal &= libs > 0
    moves = np.flatnonzero(legal.reshape(-1)).tolist()
    if variant != "pass_not_legal":
        moves.append(cells)
    seq = ([cells] * int(root_passes) if variant != "passes_no_root" else []) + list(path_actions)
    if variant == "passes_any_two":
        two = seq.count(cells) >= 2
    else:
        two = len(seq) >= 2 and seq[-1] == cells and seq[-2] == cells
    full = not empty.any() and variant != "full_not_terminal"
    checked = len(path_actions) >= 1 or variant == "root_terminal"
    return moves, bool(checked and (two or full))


def board_legal(root_empty, path_actions, pass_action=None):
    taken = {a for a in path_actions if a != pass_action}
    return [a for a in root_empty if a not in taken]


def np_wave(tree: NpTree, W: int, max_depth: int, legal_of, pol_rows, vals, policy="full",
            noise=None, eps=0.0, root_positive=False, terminal_of=None):
    """One wave: W sequential select_paths, unique leaves in first-occurrence order evaluated
    from pol_rows/vals (row u for the u-th unique leaf), expansion, then backup in order.
    terminal_of(path actions), when given, names the terminal leaves, which are evaluated and
    backed up but not expanded (optimized_wave_search.py:374-376); the root never is."""
    tree.wave_refused = False
    paths = [tree.select_path(max_depth) for _ in range(W)]
    leaves = [p[-1] for p in paths]
    uniq = []
    for l in leaves:
        if l not in uniq:
            uniq.append(l)
    for u, leaf in enumerate(uniq):
        if tree.expanded[leaf]:
            continue
        path = paths[leaves.index(leaf)]
        pacts = [int(tree.action[x]) for x in path[1:]]
        if terminal_of is not None and pacts and terminal_of(pacts):
            continue
        legal = legal_of(pacts)
        if not legal:
            continue
        root_visits = int(tree.N[0]) - tree.vli * W
        acts, pri = choose_children(legal, pol_rows[u], leaf == 0, policy, root_visits, noise, eps)
        if len(acts) <= 512:
            tree.expand(leaf, acts, pri)
    for s, path in enumerate(paths):
        tree.backup(path, vals[uniq.index(leaves[s])], root_positive)
    return paths, uniq


def grouped_select(tree: NpTree, W: int, max_depth: int):
    """The device schedule of the selection, restated: level by level, the simulations at one
    node form a group processed in simulation order, the r-th member seeing Np = N[p] + VL*r
    and each child c with N[c] + VL*(members before it that chose c).  N is then advanced by
    VL per path entry.  Returns the paths; must equal W sequential select_paths."""
    paths = [[0] for _ in range(W)]
    groups = {0: list(range(W))}
    depth = 0
    base = tree.N.copy()
    while groups:
        nxt = {}
        for p, members in groups.items():
            leaf = (not tree.expanded[p]) or tree.nchild[p] == 0 or depth == max_depth - 1
            if leaf:
                continue
            extra = {}
            saved = {}
            f, k = int(tree.first[p]), int(tree.nchild[p])
            for i in range(k):
                saved[int(tree.children[f + i])] = int(tree.N[int(tree.children[f + i])])
            for r, s in enumerate(members, start=1):
                for c, n0 in saved.items():
                    tree.N[c] = n0 + tree.vli * extra.get(c, 0)
                c = tree.best_child(p, int(base[p]) + tree.vli * r)
                if c < 0:
                    continue
                extra[c] = extra.get(c, 0) + 1
                paths[s].append(c)
                nxt.setdefault(c, []).append(s)
            for c, n0 in saved.items():
                tree.N[c] = n0
        groups = nxt
        depth += 1
    for path in paths:
        for x in path:
            tree.N[x] += tree.vli
    return paths


def overlap_select(tree: NpTree, W: int, max_depth: int, block: int = 64):
    """The level overlap of the device schedule, restated.  The root's chain runs over all W
    members without touching the children's N.  Its members are then taken in blocks of
    `block` simulations: for each block, each root child c continues its chain with the
    block's members of c, N[c] growing by VL per member and each picked child's N by VL per
    pick, in place, so that the next block of c sees them.  Deeper levels run as in
    grouped_select, the level-2 nodes already holding their members' virtual loss.  Returns
    the paths; must equal W sequential select_paths."""
    vli = tree.vli
    if (not tree.expanded[0]) or tree.nchild[0] == 0 or max_depth <= 1:
        return grouped_select(tree, W, max_depth)
    paths = [[0] for _ in range(W)]

    def chain(p, np0, m, persist):
        """picks of p's m members in order; the children's N keep the picks' VL if persist"""
        f, k = int(tree.first[p]), int(tree.nchild[p])
        saved = {int(tree.children[f + i]): int(tree.N[int(tree.children[f + i])])
                 for i in range(k)}
        extra, picks = {}, []
        for r in range(1, m + 1):
            for c, n in saved.items():
                tree.N[c] = n + vli * extra.get(c, 0)
            c = tree.best_child(p, np0 + vli * r)
            picks.append(c)
            if c >= 0:
                extra[c] = extra.get(c, 0) + 1
        for c, n in saved.items():
            tree.N[c] = n + (vli * extra.get(c, 0) if persist else 0)
        return picks

    n_root = int(tree.N[0])
    root_pick = chain(0, n_root, W, persist=False)
    tree.N[0] = n_root + vli * W
    pick1 = [-1] * W
    for b0 in range(0, W, block):
        members_of = {}
        for s in range(b0, min(W, b0 + block)):
            if root_pick[s] >= 0:
                members_of.setdefault(root_pick[s], []).append(s)
        for c, mem in members_of.items():
            np0 = int(tree.N[c])
            tree.N[c] = np0 + vli * len(mem)
            if (not tree.expanded[c]) or tree.nchild[c] == 0 or max_depth <= 2:
                continue
            for s, x in zip(mem, chain(c, np0, len(mem), persist=True)):
                pick1[s] = x
    groups = {}
    for s in range(W):
        if root_pick[s] >= 0:
            paths[s].append(root_pick[s])
            if pick1[s] >= 0:
                paths[s].append(pick1[s])
                groups.setdefault(pick1[s], []).append(s)
    depth = 2
    while groups:
        nxt = {}
        for p, members in groups.items():
            if (not tree.expanded[p]) or tree.nchild[p] == 0 or depth == max_depth - 1:
                continue
            np0 = int(tree.N[p]) - (vli * len(members) if depth == 2 else 0)
            for s, c in zip(members, chain(p, np0, len(members), persist=False)):
                if c >= 0:
                    paths[s].append(c)
                    nxt.setdefault(c, []).append(s)
        groups = nxt
        depth += 1
    for path in paths:
        for x in path[3:]:
            tree.N[x] += vli
    return paths


RUNAHEAD_VARIANTS = ("resume_without_counts", "resume_parent_count_restarted")


def runahead_select(tree: NpTree, W: int, max_depth: int, budgets: dict, done: dict,
                    variant=None):
    """The run-ahead of level-1 chains (512-thread select kernels), restated.  Before the root
    chain, root child c (a key of budgets) runs its own chain for budgets[c] ranks from the
    wave's start state (N of c and of c's children as they are), recording its picks; done[c]
    <= budgets[c] is how many of those ranks it finished (a chain stopped early).  After the
    root chain, c's level-1 group of m members takes the record's first m picks when done[c] >=
    m; otherwise it takes the done[c] recorded picks and continues the chain from rank done[c]
    with those picks' virtual loss on the children; groups without a record run their chain.
    Deeper levels as grouped_select.  Returns the paths; must equal W sequential select_paths.
    variant: "resume_without_counts" continues without the recorded picks' virtual loss;
    "resume_parent_count_restarted" continues with the parent count of rank 0 at rank done[c]."""
    vli = tree.vli
    if (not tree.expanded[0]) or tree.nchild[0] == 0 or max_depth <= 2:
        return grouped_select(tree, W, max_depth)

    def chain(p, np0, m, start=()):
        """picks of ranks len(start)..m-1 of p's chain, the picks `start` already made"""
        f, k = int(tree.first[p]), int(tree.nchild[p])
        saved = {int(tree.children[f + i]): int(tree.N[int(tree.children[f + i])])
                 for i in range(k)}
        extra, picks = {}, list(start)
        if variant != "resume_without_counts":
            for c in start:
                if c >= 0:
                    extra[c] = extra.get(c, 0) + 1
        for r in range(len(start) + 1, m + 1):
            for c, n in saved.items():
                tree.N[c] = n + vli * extra.get(c, 0)
            rr = r - len(start) if variant == "resume_parent_count_restarted" else r
            c = tree.best_child(p, np0 + vli * rr)
            picks.append(c)
            if c >= 0:
                extra[c] = extra.get(c, 0) + 1
        for c, n in saved.items():
            tree.N[c] = n
        return picks

    records = {}
    for c, M in budgets.items():
        if tree.expanded[c] and tree.nchild[c] > 0:
            records[c] = chain(c, int(tree.N[c]), M)[:done[c]]
    n_root = int(tree.N[0])
    root_pick = chain(0, n_root, W)
    tree.N[0] = n_root + vli * W
    members = {}
    for s in range(W):
        if root_pick[s] >= 0:
            members.setdefault(root_pick[s], []).append(s)
    for c in members:  # the level-1 nodes' virtual loss
        tree.N[c] += vli * len(members[c])
    paths = [[0] for _ in range(W)]
    groups = {}
    for c, mem in members.items():
        for s in mem:
            paths[s].append(c)
        if (not tree.expanded[c]) or tree.nchild[c] == 0:
            continue
        np0 = int(tree.N[c]) - vli * len(mem)
        m = len(mem)
        rec = records.get(c)
        if rec is not None and len(rec) >= m:
            picks = rec[:m]
        elif rec is not None:
            picks = chain(c, np0, m, start=rec)
        else:
            picks = chain(c, np0, m)
        for s, x in zip(mem, picks):
            if x >= 0:
                paths[s].append(x)
                groups.setdefault(x, []).append(s)
    depth = 2
    while groups:
        nxt = {}
        for p, mem in groups.items():
            if (not tree.expanded[p]) or tree.nchild[p] == 0 or depth == max_depth - 1:
                continue
            for s, x in zip(mem, chain(p, int(tree.N[p]), len(mem))):
                if x >= 0:
                    paths[s].append(x)
                    nxt.setdefault(x, []).append(s)
        groups = nxt
        depth += 1
    for path in paths:
        for x in path[2:]:
            tree.N[x] += vli
    return paths


def fused_ucb_selection(node_indices, children_start, children_end, children, q_values,
                        visit_counts, priors, c_puct):
    """mcts::fused_ucb_selection as its CUDA kernel computes it
    (python/mcts/gpu/mcts_kernels.cu:1466-1512), in float32: for parent p and row
    [start, end), ucb_i = (n_i > 0 ? q[c_i] : 0) + ((c * P_i) * sqrtf(N_p)) / (1 + n_i), and the
    row position of the first ucb above -1e10 (strict '>'), or -1 for an empty row."""
    F = np.float32
    c = F(c_puct)
    out = np.full(len(node_indices), -1, np.int32)
    for b, p in enumerate(node_indices):
        start, end = int(children_start[p]), int(children_end[p])
        if start >= end:
            continue
        sp = np.sqrt(F(visit_counts[p]))
        best, arg = F(-1e10), -1
        for i in range(start, end):
            ch = int(children[i])
            n = int(visit_counts[ch])
            q = F(q_values[ch]) if n > 0 else F(0.0)
            ucb = F(q + F(F(F(c * F(priors[i])) * sp) / F(F(1.0) + F(n))))
            if ucb > best:
                best, arg = ucb, i - start
        out[b] = arg
    return out


# ---- the reference accelerator's remaining operators (mcts_gpu_accelerator.py:81-207) ----------
# Trees of the reference's GPU variant: a dense children table [num_nodes, max_children] whose
# rows end at the first negative entry, per-node arrays, CSR edges.  Sequential float32 loops,
# in the order the reference's kernels take their elements.

def _row(children, node):
    """The children of `node` up to the row's first negative entry (or the first entry past the
    table's rows, which the HIP operators take as the row's end)."""
    out = []
    for c in children[node]:
        c = int(c)
        if c < 0 or c >= children.shape[0]:
            break
        out.append(c)
    return out


def find_expansion_nodes(current_nodes, valid_mask, wave_size, children, visit_counts):
    """find_expansion_nodes_kernel (python/mcts/gpu/mcts_kernels.cu:46-87): for path s <
    wave_size with valid_mask[s] and 0 <= node < num_nodes, the node when no entry of its table
    row is >= 0 and its visit count is 0; listed here in path order."""
    out = []
    for s in range(wave_size):
        node = int(current_nodes[s])
        if not valid_mask[s] or node < 0 or node >= children.shape[0]:
            continue
        if not (children[node] >= 0).any() and int(visit_counts[node]) == 0:
            out.append(node)
    return np.array(out, np.int32)


def batched_ucb_selection(q_values, visit_counts, parent_visits, priors, row_ptr, col_indices,
                          c_puct):
    """batched_ucb_selection_kernel (mcts_kernels.cu:240-318) for each row b: (selected, score).
    sqrt_parent = sqrtf((float)parent_visits[b] + 1); ucb_i = (n_i > 0 ? q[c_i] : 0) +
    ((c * P_i) * sqrt_parent) / (1 + n_i) over edges i with c_i >= 0 (and, as the HIP operator
    bounds them, i and c_i below the number of children); the first maximum above -1e10
    (position 0 / score -1e10 without one), -1 / 0 for an empty row, 0 / 0 for a negative start
    or a decreasing row."""
    nc = len(q_values)
    c = F(c_puct)
    B = len(parent_visits)
    sel = np.zeros(B, np.int32)
    sc = np.zeros(B, np.float32)
    for b in range(B):
        start, end = int(row_ptr[b]), int(row_ptr[b + 1])
        if start < 0 or end < start:
            continue
        if start == end:
            sel[b] = -1
            continue
        sp = np.sqrt(F(F(parent_visits[b]) + F(1.0)))
        best, arg = F(-1e10), 0
        for i in range(start, min(end, nc)):
            ch = int(col_indices[i])
            if ch < 0 or ch >= nc:
                continue
            n = F(visit_counts[ch])
            q = F(q_values[ch]) if n > 0 else F(0.0)
            ucb = F(q + F(F(F(c * F(priors[i])) * sp) / F(F(1.0) + n)))
            if ucb > best:
                best, arg = ucb, i - start
        sel[b], sc[b] = arg, best
    return sel, sc


def fused_select_expand(roots, children, visit_counts, q_values, prior_probs, is_expanded,
                        max_depth, c_puct):
    """fused_select_expand_kernel (mcts_kernels.cu:451-544): (paths [W, max_depth],
    path_lengths, expand_nodes, needs_expansion).  From the root, while depth < max_depth - 1:
    an expanded node scores its children, +inf when unvisited, else q[c] + ((c_puct * P[c]) *
    sqrtf((float)N[node])) / (1 + n); the first maximum above -inf is next.  A node that is not
    expanded or has no such child ends the path (expansion at depth + 1); a path that reaches
    the depth limit reports 0, 0, False."""
    c = F(c_puct)
    W, nn = len(roots), children.shape[0]
    paths = np.full((W, max_depth), -1, np.int32)
    plen = np.zeros(W, np.int32)
    exp = np.zeros(W, np.int32)
    need = np.zeros(W, np.bool_)
    for w in range(W):
        node = int(roots[w])
        path = [node]
        leaf = node < 0 or node >= nn
        while not leaf and len(path) - 1 < max_depth - 1:
            nxt = -1
            if is_expanded[node]:
                sp = np.sqrt(F(visit_counts[node]))
                best = F(-np.inf)
                for ch in _row(children, node):
                    n = int(visit_counts[ch])
                    if n == 0:
                        u = F(np.inf)
                    else:
                        u = F(F(q_values[ch]) + F(F(F(c * F(prior_probs[ch])) * sp) /
                                                  F(F(1.0) + F(n))))
                    if u > best:
                        best, nxt = u, ch
            if nxt < 0:
                leaf = True
                break
            node = nxt
            path.append(node)
        paths[w, :len(path)] = path
        if leaf:
            plen[w], exp[w], need[w] = len(path), node, True
    return paths, plen, exp, need


def _rsqrt_of_rcp(pv):
    """1 / sqrt(r), r = 1 / (float)(pv + 1) in float32, the square root and its reciprocal in
    float64, rounded once to float32."""
    r = F(F(1.0) / F(pv + 1))
    return F(1.0 / np.sqrt(np.float64(r)))


def fused_select_expand_optimized(roots, children, visit_counts, value_sums, priors, max_depth,
                                  c_puct):
    """fused_select_expand_optimized_kernel (mcts_kernels.cu:546-640): (paths, path_lengths,
    ucb_scores).  While depth < max_depth - 1 and depth < 32: a node without visits ends the
    path; its children score q + ((c_puct * P[c]) * sqrt_parent) * (1 / (1 + n)), q = n > 0 ?
    W[c] * (1 / (n + 1e-8)) : 0 (float32 reciprocals, sqrt_parent as _rsqrt_of_rcp); the first
    maximum above -inf is next, and none ends the path.  path_lengths = depth + 1; ucb_scores
    holds the root's row of scores (0 elsewhere)."""
    c = F(c_puct)
    W, nn = len(roots), children.shape[0]
    mc = children.shape[1]
    paths = np.full((W, max_depth), -1, np.int32)
    plen = np.zeros(W, np.int32)
    ucb = np.zeros((W, mc), np.float32)
    for w in range(W):
        node = int(roots[w])
        path = [node]
        if 0 <= node < nn:
            while len(path) - 1 < max_depth - 1 and len(path) - 1 < 32:
                pv = int(visit_counts[node])
                if pv == 0:
                    break
                sp = _rsqrt_of_rcp(pv)
                best, nxt = F(-np.inf), -1
                for i, ch in enumerate(_row(children, node)):
                    n = int(visit_counts[ch])
                    q = F(F(value_sums[ch]) * F(F(1.0) / F(F(n) + F(1e-8)))) if n > 0 else F(0)
                    u = F(q + F(F(F(c * F(priors[ch])) * sp) * F(F(1.0) / F(F(1.0) + F(n)))))
                    if len(path) == 1:
                        ucb[w, i] = u
                    if u > best:
                        best, nxt = u, ch
                if nxt < 0:
                    break
                node = nxt
                path.append(node)
        paths[w, :len(path)] = path
        plen[w] = len(path)
    return paths, plen, ucb


def _wrap32(x):
    return np.int32((x + 2**31) % 2**32 - 2**31)


def batched_add_children(parent_indices, actions, priors, num_children, tree, max_nodes,
                         max_children, max_edges):
    """batched_add_children_kernel (mcts_kernels.cu:1122-1189) with the items taken in batch
    order.  tree: dict of numpy arrays node_counter [1], edge_counter [1], children [max_nodes *
    max_children], parent_indices_out, parent_actions_out, node_priors_out, visit_counts_out,
    value_sums_out [max_nodes], col_indices, edge_actions, edge_priors [max_edges], updated in
    place.  Returns child_indices [batch * max_children] (-1 where nothing is written)."""
    B = len(parent_indices)
    out = np.full(B * max_children, -1, np.int32)
    for b in range(B):
        p, n = int(parent_indices[b]), int(num_children[b])
        if p < 0 or p >= max_nodes or n <= 0:
            continue
        nd, ed = int(tree["node_counter"][0]), int(tree["edge_counter"][0])
        tree["node_counter"][0] = _wrap32(nd + n)   # int32 atomics wrap
        tree["edge_counter"][0] = _wrap32(ed + n)
        if nd < 0 or ed < 0 or nd + n > max_nodes or ed + n > max_edges:
            continue
        for i in range(min(n, max_children)):
            ch, e = nd + i, ed + i
            a, pr = actions[b * max_children + i], priors[b * max_children + i]
            tree["parent_indices_out"][ch] = p
            tree["parent_actions_out"][ch] = a
            tree["node_priors_out"][ch] = pr
            tree["visit_counts_out"][ch] = 0
            tree["value_sums_out"][ch] = 0.0
            tree["children"][p * max_children + i] = ch
            tree["col_indices"][e] = ch
            tree["edge_actions"][e] = a
            tree["edge_priors"][e] = pr
            out[b * max_children + i] = ch
    return out


# ---- more operators of the reference's pybind module (mcts_kernels.cu:2342-2410) -----------
# Sequential loops in the order the reference's kernels visit their elements.  Each takes a
# `variant` naming a planted misreading, used only by the tests that show the known answers
# fail on it; None is the operator.

PSVL_VARIANTS = (
    "sqrt_no_plus1",      # sqrt(N_parent) instead of sqrt(N_parent + 1)
    "parent_with_vl",     # the parent's virtual-loss count added to its visits
    "value_without_vl",   # W without VL * virtual_loss_value
    "row_ends_at_neg",    # the row ends at its first negative entry instead of skipping it
    "mask_at_root",       # the legal filter applied at node 0 too
    "vl_between_sims",    # each selection's virtual loss seen by the later simulations
)


def parallel_select_with_virtual_loss(parent_nodes, children, visit_counts, vl_counts,
                                      value_sums, priors, child_actions, c_puct, vl_value,
                                      legal_masks=None, variant=None):
    """parallel_select_with_virtual_loss_kernel (mcts_kernels.cu:962-1053) for every simulation
    from the same counts, then +1 virtual loss per selection (:1990-1996).  priors: [nodes] or
    per simulation [sims, stride].  Returns (selected, virtual-loss counts after)."""
    if variant is not None and variant not in PSVL_VARIANTS:
        raise ValueError(f"unknown variant {variant!r}")
    children = np.asarray(children)
    vl = np.array(vl_counts, np.int32)
    nn = len(visit_counts)
    per_sim = np.ndim(priors) == 2
    out = []
    c_puct, vlv = F(c_puct), F(vl_value)
    for s, p in enumerate(parent_nodes):
        p = int(p)
        if p < 0 or p >= children.shape[0] or p >= nn:
            out.append(-1)
            continue
        pv = int(visit_counts[p]) + (int(vl[p]) if variant == "parent_with_vl" else 0)
        sq = F(math.sqrt(float(F(pv if variant == "sqrt_no_plus1" else pv + 1))))
        best, arg = F(-np.inf), -1
        for c in children[p]:
            c = int(c)
            if c < 0 and variant == "row_ends_at_neg":
                break
            if c < 0 or c >= nn:
                continue
            if legal_masks is not None and (p != 0 or variant == "mask_at_root"):
                a = int(child_actions[c])
                if 0 <= a < legal_masks.shape[1] and not legal_masks[s, a]:
                    continue
            if per_sim:
                if c >= priors.shape[1]:
                    continue
                prior = F(priors[s, c])
            else:
                prior = F(priors[c])
            n = int(visit_counts[c]) + int(vl[c])
            w = F(value_sums[c]) if variant == "value_without_vl" else \
                F(F(value_sums[c]) + F(F(int(vl[c])) * vlv))
            q = F(w / F(n)) if n > 0 else F(0.0)
            ucb = F(q + F(F(F(c_puct * prior) * sq) / F(F(1.0) + F(n))))
            if ucb > best:
                best, arg = ucb, c
        out.append(arg)
        if variant == "vl_between_sims" and arg >= 0:
            vl[arg] += 1
    if variant != "vl_between_sims":
        for c in out:
            if 0 <= c < len(vl):
                vl[c] += 1
    return np.array(out, np.int32), vl


UCBN_VARIANTS = (
    "prior_unmixed",     # the noise left out of the prior
    "none_is_minus1",    # -1 instead of 0 when no score is above -1e10
    "q_zero_unvisited",  # q = 0 for an unvisited child
)


def fused_ucb_with_noise(q_values, visit_counts, priors, noise, parent_visits_sqrt, c_puct,
                         epsilon, variant=None):
    """fused_ucb_with_noise_kernel (mcts_kernels.cu:760-797): per simulation, the position of
    the first maximum above -1e10 of q + c (1-eps) P + eps noise) sqrt / (1 + N), else 0."""
    if variant is not None and variant not in UCBN_VARIANTS:
        raise ValueError(f"unknown variant {variant!r}")
    keep, eps = F(F(1.0) - F(epsilon)), F(epsilon)
    c, sq = F(c_puct), F(parent_visits_sqrt)
    out = []
    for s in range(noise.shape[0]):
        best, arg = F(-1e10), (-1 if variant == "none_is_minus1" else 0)
        for i in range(len(q_values)):
            mixed = F(priors[i]) if variant == "prior_unmixed" else \
                F(F(keep * F(priors[i])) + F(eps * F(noise[s, i])))
            n = int(visit_counts[i])
            q = F(0.0) if (variant == "q_zero_unvisited" and n == 0) else F(q_values[i])
            ucb = F(q + F(F(F(c * mixed) * sq) / F(F(1.0) + F(n))))
            if ucb > best:
                best, arg = ucb, i
        out.append(arg)
    return np.array(out, np.int32)


UCBD_VARIANTS = (
    "returns_slot",      # the slot position instead of the child id
    "sqrt_no_plus1",     # sqrt(pv) instead of sqrt(pv + 1)
    "value_unvisited",   # the child's value used when it has no visits
)


def batched_ucb_selection_dense(batch_children, batch_priors, parent_visits, child_visits,
                                child_values, valid_mask, c_puct, variant=None):
    """batched_ucb_selection_dense_kernel (mcts_kernels.cu:1364-1409): per item, the child of
    the first maximum above -1e10 over valid slots whose child is in [0, len(child_visits)),
    else -1."""
    if variant is not None and variant not in UCBD_VARIANTS:
        raise ValueError(f"unknown variant {variant!r}")
    c = F(c_puct)
    nv = len(child_visits)
    out = []
    for b in range(batch_children.shape[0]):
        pv = int(parent_visits[b])
        sq = F(math.sqrt(float(F(F(pv) + (F(0.0) if variant == "sqrt_no_plus1" else F(1.0))))))
        best, arg = F(-1e10), -1
        for j in range(batch_children.shape[1]):
            if not valid_mask[b, j]:
                continue
            ch = int(batch_children[b, j])
            if ch < 0 or ch >= nv:
                continue
            n = int(child_visits[ch])
            v = F(child_values[ch]) if (n > 0 or variant == "value_unvisited") else F(0.0)
            ucb = F(v + F(F(F(c * F(batch_priors[b, j])) * sq) / F(F(1.0) + F(n))))
            if ucb > best:
                best, arg = ucb, (j if variant == "returns_slot" else ch)
        out.append(arg)
    return np.array(out, np.int32)


BFS_VARIANTS = (
    "dfs",              # depth-first numbering
    "level_by_id",      # a level's new nodes numbered by old id instead of discovery order
    "last_occurrence",  # a child met twice in a level numbered at its last occurrence
)


def parallel_bfs_subtree(row_ptr, col_indices, root, max_nodes, variant=None):
    """The subtree of root in a CSR graph, numbered breadth-first (gpu_bfs.py:70-127, the
    order of a FIFO queue: levels in order, children in row order, first occurrence), children
    outside [0, max_nodes) skipped.  Returns (in_subtree, node_remap, count)."""
    if variant is not None and variant not in BFS_VARIANTS:
        raise ValueError(f"unknown variant {variant!r}")
    E = len(col_indices)

    def row(v):
        a = min(max(int(row_ptr[v]), 0), E)
        b = min(max(int(row_ptr[v + 1]), a), E)
        return [int(c) for c in col_indices[a:b]]

    ins = np.zeros(max_nodes, bool)
    remap = np.full(max_nodes, -1, np.int32)
    ins[root], remap[root] = True, 0
    order = [root]
    if variant == "dfs":
        stack = [root]
        while stack:
            v = stack.pop()
            for c in reversed(row(v)):
                if 0 <= c < max_nodes and not ins[c]:
                    ins[c] = True
                    remap[c] = len(order)
                    order.append(c)
                    stack.append(c)
        return ins, remap, len(order)
    level = [root]
    while level:
        found = []
        for v in level:
            for c in row(v):
                if 0 <= c < max_nodes and not ins[c]:
                    if variant == "last_occurrence" and c in found:
                        found.remove(c)
                    if c not in found:
                        found.append(c)
        if variant == "level_by_id":
            found = sorted(found)
        for c in found:
            ins[c] = True
            remap[c] = len(order)
            order.append(c)
        level = found
    return ins, remap, len(order)


EDGE_VARIANTS = (
    "by_new_index",     # nodes taken in new-index order instead of old-index order
    "child_outside",    # edges to children outside the subtree kept (child -1)
)


def extract_subtree_edges(row_ptr, col_indices, edge_actions, in_subtree, node_remap,
                          variant=None):
    """The subtree's edges (extract_subtree_edges_kernel, mcts_kernels.cu:2201-2244, in the
    order of one thread): nodes of the subtree in ascending old index, each row in order, edges
    whose child lies in the subtree, as (new parent, new child, action or 0)."""
    if variant is not None and variant not in EDGE_VARIANTS:
        raise ValueError(f"unknown variant {variant!r}")
    n, E = len(in_subtree), len(col_indices)
    nodes = [i for i in range(n) if in_subtree[i]]
    if variant == "by_new_index":
        nodes.sort(key=lambda i: int(node_remap[i]))
    par, chl, act = [], [], []
    for i in nodes:
        a = min(max(int(row_ptr[i]), 0), E)
        b = min(max(int(row_ptr[i + 1]), a), E)
        for e in range(a, b):
            c = int(col_indices[e])
            inside = 0 <= c < n and in_subtree[c]
            if not inside and not (variant == "child_outside" and 0 <= c < n):
                continue
            par.append(int(node_remap[i]))
            chl.append(int(node_remap[c]))
            act.append(int(edge_actions[e]) if edge_actions is not None else 0)
    return np.array(par, np.int32), np.array(chl, np.int32), np.array(act, np.int16)
