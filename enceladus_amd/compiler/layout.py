"""Wave64 bit-permutation layouts.

A tile's dimensions are powers of two, so a coordinate is a set of bits. A `Layout`
assigns each coordinate bit (dim, bit) to exactly one hardware bit: a register bit (which
element of a thread's register array), one of the 6 lane bits of a 64-wide wavefront, or
a warp (wavefront-in-workgroup) bit. Lane and warp bits that carry no coordinate bit are
broadcast: those threads hold copies. This is the reference's `BitLayout` idea
(reference: src/enceladus/compiler/layout.py:46-106, `LANE_BITS=5` at :17) restricted to
single-bit bases and re-targeted to 64 lanes (6 lane bits) and to MFMA tile layouts.

Register bit 0 is the fastest-varying register index, so `reg` bits that map to
consecutive low bits of the contiguous dimension form a vector.
"""

from __future__ import annotations

from dataclasses import dataclass

LANE_BITS = 6

Bit = tuple  # (dim, bit)


def log2(n: int) -> int:
    return n.bit_length() - 1


@dataclass(frozen=True)
class Layout:
    shape: tuple[int, ...]
    reg: tuple          # tuple[Bit, ...]
    lane: tuple         # len 6, Bit | None
    warp: tuple         # len log2(num_warps), Bit | None
    kind: str = "blocked"

    # -- basic queries ---------------------------------------------------------------
    @property
    def nregs(self) -> int:
        return 1 << len(self.reg)

    @property
    def num_warps(self) -> int:
        return 1 << len(self.warp)

    def key(self) -> tuple:
        return (self.shape, self.reg, self.lane, self.warp)

    def __hash__(self):
        return hash(self.key())

    def __eq__(self, other):
        return isinstance(other, Layout) and self.key() == other.key()

    def check(self) -> None:
        seen = set()
        for b in (*self.reg, *self.lane, *self.warp):
            if b is None:
                continue
            assert b not in seen, f"duplicate bit {b} in {self}"
            seen.add(b)
        want = {(d, i) for d, s in enumerate(self.shape) for i in range(log2(s))}
        assert seen == want, f"layout bits {sorted(seen)} != tile bits {sorted(want)}"
        assert len(self.lane) == LANE_BITS

    def reg_coord(self, r: int) -> tuple[int, ...]:
        c = [0] * len(self.shape)
        for i, b in enumerate(self.reg):
            if (r >> i) & 1:
                c[b[0]] |= 1 << b[1]
        return tuple(c)

    def thread_coord(self, lane: int, warp: int) -> tuple[int, ...]:
        c = [0] * len(self.shape)
        for i, b in enumerate(self.lane):
            if b is not None and (lane >> i) & 1:
                c[b[0]] |= 1 << b[1]
        for i, b in enumerate(self.warp):
            if b is not None and (warp >> i) & 1:
                c[b[0]] |= 1 << b[1]
        return tuple(c)

    def owns(self, lane: int, warp: int) -> bool:
        """Whether this thread is the canonical owner of its elements (broadcast bits 0)."""
        for i, b in enumerate(self.lane):
            if b is None and (lane >> i) & 1:
                return False
        for i, b in enumerate(self.warp):
            if b is None and (warp >> i) & 1:
                return False
        return True

    def has_broadcast(self) -> bool:
        return any(b is None for b in (*self.lane, *self.warp))

    def vec_dim_bits(self) -> tuple[int, int]:
        """(dim, n): register bits 0..n-1 map to bits 0..n-1 of one dim."""
        if not self.reg:
            return (len(self.shape) - 1 if self.shape else 0, 0)
        d = self.reg[0][0]
        n = 0
        while n < len(self.reg) and self.reg[n] == (d, n):
            n += 1
        return d, n

    # -- transforms -----------------------------------------------------------------
    def _map(self, f, shape, kind=None) -> "Layout":
        g = lambda b: None if b is None else f(b)  # noqa: E731
        reg = tuple(x for x in (g(b) for b in self.reg) if x is not None)
        lay = Layout(tuple(shape), reg, tuple(g(b) for b in self.lane),
                     tuple(g(b) for b in self.warp), kind or self.kind)
        return lay

    def slice(self, axis: int) -> "Layout":
        """The layout of a reduction over `axis`: its bits become broadcast."""
        shape = self.shape[:axis] + self.shape[axis + 1:]

        def f(b):
            if b[0] == axis:
                return None
            return (b[0] - (b[0] > axis), b[1])
        return self._map(f, shape, "slice")

    def expand(self, axis: int) -> "Layout":
        shape = self.shape[:axis] + (1,) + self.shape[axis:]
        return self._map(lambda b: (b[0] + (b[0] >= axis), b[1]), shape)

    def permute(self, perm: tuple[int, ...]) -> "Layout":
        inv = {p: i for i, p in enumerate(perm)}
        shape = tuple(self.shape[p] for p in perm)
        return self._map(lambda b: (inv[b[0]], b[1]), shape)

    def reshape(self, shape: tuple[int, ...]) -> "Layout":
        """The same hardware bits over a row-major reshape of the tile: with power-of-two
        dims a reshape only relabels coordinate bits (linear bit position is preserved)."""
        def table(shp):
            pos, out = 0, {}
            for d in reversed(range(len(shp))):
                for i in range(log2(shp[d])):
                    out[(d, i)] = pos + i
                pos += log2(shp[d])
            return out
        src = table(self.shape)
        back = {p: b for b, p in table(tuple(shape)).items()}
        return self._map(lambda b: back[src[b]], shape)

    def project(self, shape: tuple[int, ...]) -> "Layout":
        """Restricts to a broadcast source shape: bits of size-1 dims become broadcast."""
        def f(b):
            return None if shape[b[0]] == 1 else b
        return self._map(f, shape)

    def lift(self, shape: tuple[int, ...]) -> "Layout":
        """Extends a layout of a broadcastable shape to `shape` (new bits fill broadcast
        lane/warp slots first, then registers)."""
        missing = [(d, i) for d, s in enumerate(shape) if self.shape[d] == 1
                   for i in range(log2(s))]
        lane, warp = list(self.lane), list(self.warp)
        for slots in (lane, warp):
            for i, b in enumerate(slots):
                if b is None and missing:
                    slots[i] = missing.pop(0)
        reg = tuple(self.reg) + tuple(missing)
        return Layout(tuple(shape), reg, tuple(lane), tuple(warp), self.kind)

    def __repr__(self) -> str:
        def s(bs):
            return "[" + ",".join("_" if b is None else f"{b[0]}.{b[1]}" for b in bs) + "]"
        return f"L{self.shape}(r{s(self.reg)} l{s(self.lane)} w{s(self.warp)})"


def is_view(src: Layout, dst: Layout) -> bool:
    """Whether a value held in `src` can be read in `dst` without moving data.

    `src.shape` must broadcast to `dst.shape`. Every thread must already hold, in its
    registers, the elements `dst` asks of it.
    """
    if len(src.shape) != len(dst.shape):
        return False
    proj = dst.project(src.shape)
    if proj.lane != src.lane or proj.warp != src.warp:
        return False
    return set(proj.reg) == set(src.reg)


def reg_index_map(src: Layout, dst: Layout) -> list[tuple[int, int]]:
    """For a view, the src register index as a function of dst register index `r`:
    a list of (dst_bit, src_bit) pairs: src_index = OR of ((r >> dst_bit) & 1) << src_bit."""
    proj = dst.project(src.shape)
    pairs = []
    for j, b in enumerate(dst.reg):
        pb = proj_bit(b, src.shape)
        if pb is None:
            continue
        i = src.reg.index(pb)
        pairs.append((j, i))
    del proj
    return pairs


def proj_bit(b, shape):
    return None if shape[b[0]] == 1 else b


# -- constructors ------------------------------------------------------------------------

def blocked(shape, order, vec: int, num_warps: int) -> Layout:
    """Vectors of `vec` elements along `order[0]`, then lanes, then warps, then registers.

    `order` lists dims fastest first. Coordinate bits are handed out in that order.
    """
    shape = tuple(shape)
    bits = [(d, i) for d in order for i in range(log2(shape[d]))]
    nvec = min(log2(vec), log2(shape[order[0]])) if shape else 0
    wb = log2(num_warps)
    if len(bits) >= LANE_BITS + wb:
        # narrower vectors when the full width would leave threads holding copies: a
        # 1024-element tile over 8 waves takes 2 elements per thread, not 4 (with 4, the
        # upper four waves would load the tile a second time)
        nvec = min(nvec, len(bits) - LANE_BITS - wb)
    reg = bits[:nvec]
    rest = bits[nvec:]
    lane = rest[:LANE_BITS]
    rest = rest[LANE_BITS:]
    warp = rest[:wb]
    rest = rest[wb:]
    reg = reg + rest
    lane = lane + [None] * (LANE_BITS - len(lane))
    warp = warp + [None] * (wb - len(warp))
    lay = Layout(shape, tuple(reg), tuple(lane), tuple(warp), "blocked")
    lay.check()
    return lay


def default_order(shape) -> list[int]:
    return list(reversed(range(len(shape))))


def default_blocked(shape, num_warps: int, elem_bytes: int = 4) -> Layout:
    vec = max(1, 16 // elem_bytes)
    if not shape:
        return Layout((), (), (None,) * LANE_BITS, (None,) * log2(num_warps))
    return blocked(shape, default_order(shape), vec, num_warps)


def scan_layout(shape, axis: int, num_warps: int) -> Layout:
    """Each thread holds a contiguous run along `axis` (register bits lowest), then lanes,
    then warps: the order a serial-then-wave-then-block scan needs."""
    shape = tuple(shape)
    others = [d for d in reversed(range(len(shape))) if d != axis]
    order = [axis] + others
    bits = [(d, i) for d in order for i in range(log2(shape[d]))]
    wb = log2(num_warps)
    nthr_bits = LANE_BITS + wb
    axis_bits = log2(shape[axis])
    k = max(0, min(axis_bits, len(bits) - nthr_bits))
    reg = bits[:k]
    rest = bits[k:]
    lane = rest[:LANE_BITS]
    rest = rest[LANE_BITS:]
    warp = rest[:wb]
    rest = rest[wb:]
    reg = reg + rest
    lane = lane + [None] * (LANE_BITS - len(lane))
    warp = warp + [None] * (wb - len(warp))
    lay = Layout(shape, tuple(reg), tuple(lane), tuple(warp), "scan")
    lay.check()
    return lay


def scan_friendly(lay: Layout, axis: int) -> bool:
    """Axis bits in increasing significance: all register bits first (as the lowest
    register bits, in order), then lane bits, then warp bits."""
    locs = []
    for d_bit in range(log2(lay.shape[axis])):
        b = (axis, d_bit)
        if b in lay.reg:
            locs.append(("r", lay.reg.index(b)))
        elif b in lay.lane:
            locs.append(("l", lay.lane.index(b)))
        else:
            locs.append(("w", lay.warp.index(b)))
    rank = {"r": 0, "l": 1, "w": 2}
    for a, c in zip(locs, locs[1:]):
        if rank[a[0]] > rank[c[0]]:
            return False
        if a[0] == c[0] and a[1] > c[1]:
            return False
    nreg = sum(1 for x in locs if x[0] == "r")
    return all(locs[i] == ("r", i) for i in range(nreg))


def scan_groups(lay: Layout, axis: int):
    """For a layout a scan can run in: (run, groups) where `run` is the number of low
    register bits holding the axis's lowest bits (a contiguous run per thread), and
    `groups` the register bit positions, in increasing significance, of axis bits that
    come after every lane and warp bit of the axis (segments scanned apart and joined by
    carries). None when the axis bits are in another order. With no groups this accepts
    exactly the layouts `scan_friendly` accepts."""
    locs = []
    for d_bit in range(log2(lay.shape[axis])):
        b = (axis, d_bit)
        if b in lay.reg:
            locs.append(("r", lay.reg.index(b)))
        elif b in lay.lane:
            locs.append(("l", lay.lane.index(b)))
        else:
            locs.append(("w", lay.warp.index(b)))
    k = 0
    while k < len(locs) and locs[k] == ("r", k):
        k += 1
    rest = locs[k:]
    i = 0
    for cat in ("l", "w"):
        prev = -1
        while i < len(rest) and rest[i][0] == cat:
            if rest[i][1] < prev:
                return None
            prev = rest[i][1]
            i += 1
    groups = []
    prev = k - 1
    for c, pos in rest[i:]:
        if c != "r" or pos <= prev:
            return None
        groups.append(pos)
        prev = pos
    if groups and i == 0:
        return None     # axis bits only in registers: they are all part of the run
    return k, groups


# -- MFMA layouts -----------------------------------------------------------------------

@dataclass(frozen=True)
class MfmaShape:
    m: int      # instruction rows
    n: int      # instruction cols
    k: int      # instruction depth
    kpl: int    # k elements per lane (operand registers)
    fn: str     # ek:: wrapper name


def pick_mfma(pm: int, pn: int, bk: int, dtype_name: str) -> MfmaShape:
    """Chooses the gfx950 MFMA for a per-warp tile pm x pn and depth bk."""
    if dtype_name == "i8":
        if pm % 32 == 0 and pn % 32 == 0 and bk % 16 == 0:
            if bk % 32 == 0:
                return MfmaShape(32, 32, 32, 16, "mfma_32x32x32")
            return MfmaShape(32, 32, 16, 8, "mfma_32x32x16")
        if bk % 64 == 0:
            return MfmaShape(16, 16, 64, 16, "mfma_16x16x64")
        return MfmaShape(16, 16, 32, 8, "mfma_16x16x32")
    if dtype_name == "fp32":
        if pm % 32 == 0 and pn % 32 == 0 and bk % 2 == 0:
            return MfmaShape(32, 32, 2, 1, "mfma_32x32x2")
        return MfmaShape(16, 16, 4, 1, "mfma_16x16x4")
    if pm % 32 == 0 and pn % 32 == 0:
        if bk % 16 == 0:
            return MfmaShape(32, 32, 16, 8, "mfma_32x32x16")
        return MfmaShape(32, 32, 8, 4, "mfma_32x32x8")
    if bk % 32 == 0:
        return MfmaShape(16, 16, 32, 8, "mfma_16x16x32")
    return MfmaShape(16, 16, 16, 4, "mfma_16x16x16")


@dataclass(frozen=True)
class DotPlan:
    """How a [BM, BN] += [BM, BK] x [BK, BN] product maps onto warps and MFMAs."""

    bm: int
    bn: int
    bk: int
    wm: int      # warps along M
    wn: int      # warps along N
    wrep: int    # extra warps holding copies (when the tile is too small)
    inst: MfmaShape
    num_warps: int
    trans: bool = False   # compute C^T = B^T A^T: M on lanes in the accumulator
    korder: tuple = ()    # k-coordinate bits in operand order (reg, lane-group, k-step)

    @property
    def tm(self) -> int:
        return self.bm // self.wm // self.inst.m

    @property
    def tn(self) -> int:
        return self.bn // self.wn // self.inst.n

    @property
    def tk(self) -> int:
        return self.bk // self.inst.k


def plan_dot(bm: int, bn: int, bk: int, num_warps: int, dtype_name: str,
             dot_warps=None, trans: bool = False, korder: tuple = ()) -> DotPlan:
    wb = log2(num_warps)
    if dot_warps is not None:
        wm, wn = int(dot_warps[0]), int(dot_warps[1])
    else:
        # Split warps to keep per-warp tiles square, preferring more warps along M.
        wm, wn = 1, 1
        for _ in range(wb):
            if bm // wm >= bn // wn and bm // (wm * 2) >= 16:
                wm *= 2
            elif bn // (wn * 2) >= 16:
                wn *= 2
            elif bm // (wm * 2) >= 16:
                wm *= 2
            else:
                break
    while wm > 1 and bm // wm < 16:
        wm //= 2
    while wn > 1 and bn // wn < 16:
        wn //= 2
    if bm < 16 or bn < 16:
        raise ValueError(f"tl.dot tiles must be at least 16x16 on MFMA, got {bm}x{bn}")
    wrep = num_warps // (wm * wn)
    inst = pick_mfma(bm // wm, bn // wn, bk, dtype_name)
    if bk % inst.k:
        raise ValueError(f"tl.dot depth {bk} isn't a multiple of the MFMA depth {inst.k}")
    nk = log2(bk)
    korder = tuple(korder) if korder else tuple(range(nk))
    return DotPlan(bm, bn, bk, wm, wn, wrep, inst, num_warps, trans, korder)


def _warp_bits(plan: DotPlan, m_bits: list, n_bits: list) -> tuple:
    """Warp bits: first the M warps, then the N warps, then replicas (broadcast)."""
    out = list(m_bits[:log2(plan.wm)]) + list(n_bits[:log2(plan.wn)])
    out += [None] * (log2(plan.num_warps) - len(out))
    return tuple(out)


def mfma_acc(plan: DotPlan) -> Layout:
    """Accumulator layout [BM, BN]. Register order: the instruction's result registers
    (fastest), then N tiles, then M tiles, so each MFMA's accumulator is contiguous."""
    i = plan.inst
    if i.m == 32:
        # 32x32: lane%32 -> col, lane bit 5 -> row bit 2; regs j0,j1 -> rows 0,1;
        # j2,j3 -> rows 3,4.
        inst_reg = [(0, 0), (0, 1), (0, 3), (0, 4)]
        lane = [(1, 0), (1, 1), (1, 2), (1, 3), (1, 4), (0, 2)]
        row_inst_bits, col_inst_bits = 5, 5
    else:
        # 16x16: lane%16 -> col, lane bits 4,5 -> row bits 2,3; regs j0,j1 -> rows 0,1.
        inst_reg = [(0, 0), (0, 1)]
        lane = [(1, 0), (1, 1), (1, 2), (1, 3), (0, 2), (0, 3)]
        row_inst_bits, col_inst_bits = 4, 4
    if plan.trans:
        # The instruction produces C^T: its rows are our columns and vice versa.
        sw = lambda b: (1 - b[0], b[1])  # noqa: E731
        inst_reg = [sw(b) for b in inst_reg]
        lane = [sw(b) for b in lane]
    tm_bits = [(0, row_inst_bits + t) for t in range(log2(plan.tm))]
    tn_bits = [(1, col_inst_bits + t) for t in range(log2(plan.tn))]
    m_w = [(0, row_inst_bits + log2(plan.tm) + t) for t in range(log2(plan.wm))]
    n_w = [(1, col_inst_bits + log2(plan.tn) + t) for t in range(log2(plan.wn))]
    reg = tuple(inst_reg + tn_bits + tm_bits)
    lay = Layout((plan.bm, plan.bn), reg, tuple(lane), _warp_bits(plan, m_w, n_w), "mfma_acc")
    lay.check()
    return lay


def mfma_operand(plan: DotPlan, which: str) -> Layout:
    """Operand layouts. A is [BM, BK] (dim 0 = M rows), B is [BK, BN] (dim 1 = N cols).

    Per lane, `kpl` consecutive k values sit in consecutive registers; lane%m (or %n)
    selects the row (col); the upper lane bits select the k group. Register order:
    k within lane, then k steps, then M (or N) tiles.
    """
    i = plan.inst
    kb = log2(i.kpl)                 # k bits held in registers per lane
    row_bits = log2(i.m)             # lane bits for the row/col index
    kgroup_bits = LANE_BITS - row_bits  # lane bits for k groups
    ko = plan.korder
    if which == "a":
        kdim, rdim = 1, 0
        tiles, wr = plan.tm, plan.wm
    else:
        kdim, rdim = 0, 1
        tiles, wr = plan.tn, plan.wn
    lane = [(rdim, t) for t in range(row_bits)]
    lane += [(kdim, ko[kb + t]) for t in range(kgroup_bits)]
    inst_k_bits = log2(i.k)
    reg = [(kdim, ko[t]) for t in range(kb)]
    reg += [(kdim, ko[inst_k_bits + t]) for t in range(log2(plan.tk))]
    reg += [(rdim, row_bits + t) for t in range(log2(tiles))]
    r_w = [(rdim, row_bits + log2(tiles) + t) for t in range(log2(wr))]
    # Warps: M warps first then N warps; an operand is shared by the other group.
    wbits = []
    for t in range(log2(plan.wm)):
        wbits.append(r_w[t] if which == "a" else None)
    for t in range(log2(plan.wn)):
        wbits.append(r_w[t] if which == "b" else None)
    wbits += [None] * (log2(plan.num_warps) - len(wbits))
    shape = (plan.bm, plan.bk) if which == "a" else (plan.bk, plan.bn)
    lay = Layout(shape, tuple(reg), tuple(lane), tuple(wbits), f"mfma_{which}")
    lay.check()
    return lay


def tr16_source(lay: Layout):
    """The address layout for reading the 16-bit fragment `lay` of a row-major [rows, cols]
    LDS tile with ds_read_b64_tr_b16, or None when `lay` does not fit that instruction.

    In each group of 16 lanes, ds_read_b64_tr_b16 gives output lane L, value t, element L % 4
    of the 8-byte read made by lane 4t + L // 4. So a register run of 4 (values t = 0..3)
    must hold 4 rows, and output lanes 0..3 must hold 4 consecutive columns: the lane that
    reads for (t, L // 4) supplies row k(t) and the first of the 4 columns of lanes
    4 (L // 4) + 0..3. The returned layout maps those address lanes (bits 0,1 <- output lane
    bits 2,3; bits 2,3 <- value t; bits 4,5 <- output lane bits 4,5) and the run index
    (register bits) to (row, column) coordinates."""
    if len(lay.shape) != 2 or len(lay.reg) < 2:
        return None
    if lay.reg[0][0] != 0 or lay.reg[1][0] != 0:
        return None
    if lay.lane[0] != (1, 0) or lay.lane[1] != (1, 1):
        return None
    if any(b is None or b[0] != 1 for b in lay.lane[2:4]):
        return None
    lane = (lay.lane[2], lay.lane[3], lay.reg[0], lay.reg[1], lay.lane[4], lay.lane[5])
    src = Layout(lay.shape, tuple(lay.reg[2:]), lane, lay.warp, "tr16")
    if not tr16_check(lay, src):
        return None
    return src


def tr16_check(lay: Layout, src: Layout) -> bool:
    """Every output lane/value of the transpose read at `src` addresses equals `lay`."""
    for w in range(lay.num_warps):
        for run in range(lay.nregs // 4):
            for ln in range(64):
                for t in range(4):
                    tc = lay.thread_coord(ln, w)
                    rc = lay.reg_coord(run * 4 + t)
                    want = (tc[0] | rc[0], tc[1] | rc[1])
                    prov = 16 * (ln // 16) + 4 * t + (ln % 16) // 4
                    ptc = src.thread_coord(prov, w)
                    prc = src.reg_coord(run)
                    got = (ptc[0] | prc[0], (ptc[1] | prc[1]) + ln % 4)
                    if got != want:
                        return False
    return True
