"""LDS layouts for staged dot operands, chosen by a bank-conflict model.

A staged tile has `lines` lines of `length` 2-byte elements. Inside a line, the element at
logical position `pos` goes to storage position `sigma(pos)` (a permutation of the
position's bits, so that a lane's MFMA fragment is one contiguous 16-byte run even when the
operand's k order interleaves lanes and registers). Lines shorter than 64 elements are
packed `k = 64 / length` to a row, so that every row spans all 32 banks; the 16-byte chunk
index inside a row is then XOR-swizzled by a function of the row:

    row = line // k,  vp = (line % k) * length + sp
    offset(line, sp) = row * pitch + (vp ^ (h(row) << (3 + csh))),
    h(row) = ((row >> sa) ^ (row >> sb)) & mask

(`csh` > 0 moves whole groups of 2^csh chunks, which transpose reads of 4 rows need.)

Bank model (gfx950 LDS, measured with SQ_LDS_BANK_CONFLICT on access-pattern kernels): a
read is served 256 bytes per cycle (64 banks of 4 bytes): 16 lanes per pass for 16-byte
reads, 32 lanes for 8-byte reads. A write is served 128 bytes per cycle: 8 lanes per pass
for 16-byte writes. A pass takes as many cycles as the largest number of distinct dwords
that fall on one bank (lanes reading the same dword share it). The chooser simulates every
store the stage loader issues and every fragment read the dot issues and keeps the
cheapest candidate; ties go to no swizzle, then to the smaller pitch.
"""

from __future__ import annotations

from dataclasses import dataclass

READ_BYTES = 256    # bytes per read pass (64 banks)
WRITE_BYTES = 128   # bytes per write pass
BANK_BYTES = 4
NO_SHIFT = 31  # `line >> 31` is 0 for every line index, so (a, 31) is a single-shift hash


@dataclass(frozen=True)
class StageLayout:
    lines: int
    length: int          # logical elements per line
    pitch: int           # elements per row in LDS (>= row length)
    mask: int = 0
    sa: int = 0
    sb: int = NO_SHIFT
    sigma: tuple = ()    # sigma[i] = storage bit of logical position bit i
    rowlen: int = 64     # lines shorter than this are packed to rows of `rowlen` elements
    csh: int = 0         # the swizzle XORs chunk groups of 2^csh chunks

    @property
    def k(self) -> int:
        """Lines per row."""
        return max(1, self.rowlen // self.length)

    @property
    def rows(self) -> int:
        return -(-self.lines // self.k)

    @property
    def elems(self) -> int:
        return self.rows * self.pitch

    def sp(self, pos: int) -> int:
        """Storage position of logical position `pos`."""
        out = 0
        for i, s in enumerate(self.sigma):
            if (pos >> i) & 1:
                out |= 1 << s
        return out

    def logical(self, sp: int) -> int:
        """Inverse of `sp`."""
        out = 0
        for i, s in enumerate(self.sigma):
            if (sp >> s) & 1:
                out |= 1 << i
        return out

    def h(self, row: int) -> int:
        return ((row >> self.sa) ^ (row >> self.sb)) & self.mask

    def offset(self, line: int, sp: int) -> int:
        row, vp = line // self.k, (line % self.k) * self.length + sp
        return row * self.pitch + (vp ^ (self.h(row) << (3 + self.csh)))

    def cexpr(self, line: str, sp: str) -> str:
        """C++ element offset for the line and storage-position expressions."""
        lsh = self.k.bit_length() - 1  # lines per row = 2^lsh
        lensh = self.length.bit_length() - 1
        return (f"ek::swz<{self.pitch}, {self.mask}, {self.sa}, {self.sb}, {lsh}, {lensh}, "
                f"{self.csh}>({line}, {sp})")


def identity_sigma(length: int) -> tuple:
    return tuple(range(length.bit_length() - 1))


def fragment_sigma(length: int, lead: list[int]) -> tuple:
    """The permutation that puts the logical bits `lead` (the position bits a lane's first
    registers carry, in register order) at storage bits 0.. and keeps the other bits in
    increasing order above them."""
    nb = length.bit_length() - 1
    rest = [b for b in range(nb) if b not in lead]
    order = list(lead) + rest            # storage bit s holds logical bit order[s]
    sigma = [0] * nb
    for s, b in enumerate(order):
        sigma[b] = s
    return tuple(sigma)


def pass_cycles(addrs: list, width: int, write: bool = False) -> int:
    """Cycles of one wave access: `addrs` holds 64 byte addresses (None = inactive lane)."""
    span = WRITE_BYTES if write else READ_BYTES
    group = span // width
    banks_n = span // BANK_BYTES
    total = 0
    for g0 in range(0, len(addrs), group):
        banks: dict[int, set] = {}
        for a in addrs[g0:g0 + group]:
            if a is None:
                continue
            for w in range(width // BANK_BYTES):
                dw = a // BANK_BYTES + w
                banks.setdefault(dw % banks_n, set()).add(dw)
        if banks:
            total += max(len(s) for s in banks.values())
    return total


def cost(lay: StageLayout, accesses: list) -> int:
    """Total cycles of `accesses`: (width_bytes, [(line, sp) | None] * 64, is_write)."""
    tot = 0
    for width, lanes, write in accesses:
        addrs = [None if x is None else 2 * lay.offset(*x) for x in lanes]
        tot += pass_cycles(addrs, width, write)
    return tot


def ideal(accesses: list) -> int:
    """Cycles of `accesses` with no bank conflict: one per pass."""
    tot = 0
    for w, lanes, write in accesses:
        g = (WRITE_BYTES if write else READ_BYTES) // w
        tot += sum(1 for g0 in range(0, len(lanes), g) if any(x is not None for x in lanes[g0:g0 + g]))
    return tot


def candidates(lines: int, length: int, sigma: tuple) -> list[StageLayout]:
    out = []
    for rl in (64, 128):
        rowlen = max(length, rl)
        if out and rowlen == out[0].rowlen:
            continue
        out += [StageLayout(lines, length, rowlen + 8, sigma=sigma, rowlen=rowlen),
                StageLayout(lines, length, rowlen, sigma=sigma, rowlen=rowlen)]
        for csh in (0, 1, 2):
            m = (min(rowlen // 8, 16) >> csh) - 1
            if m <= 0:
                continue
            for a in range(5):
                out.append(StageLayout(lines, length, rowlen, m, a, NO_SHIFT, sigma, rowlen, csh))
            for a in range(4):
                for b in range(a + 1, 7):
                    out.append(StageLayout(lines, length, rowlen, m, a, b, sigma, rowlen, csh))
    return out


def choose(lines: int, length: int, sigma: tuple, accesses: list) -> tuple[StageLayout, int]:
    best = None
    for i, c in enumerate(candidates(lines, length, sigma)):
        k = (cost(c, accesses), c.mask != 0, c.pitch, i)
        if best is None or k < best[0]:
            best = (k, c)
    return best[1], best[0][0]
