"""CPU emulation of the GEMM engine's LDS refill addressing (csrc/ffn_gemm.hpp, Engine::issue_one
and Engine::issue_one_fast), for every compiled tile variant and for the waves each kernel form
lets issue the refill.

The refill of one LDS stage is split into 1 KiB DMA blocks (64 lanes x 16 bytes); the issuing
wave w sends A blocks w * A_PW + D and B blocks w * B_PW + (D - A_PW).  Only waves [0, DW) may
issue: a wave past DW computes blocks past the tile, i.e. rows past BM (BN) of the operand and
LDS bytes past the stage.  On the SALU-addressed refill those rows travel in soffset, which the
buffer range check does not cover, so for the last tile row or column they are reads past the
operand's allocation.

The second half of this file replays the schedule of the single-launch FFN kernel that was built
and removed (it faulted on its first GPU run, on the aligned mid-size FFN with the eight-wave
256x256 up tile and the K-sliced eight-wave 128x128 down tile, 256 workgroups).  That kernel
constructed both GEMM engines with the refill role on for every wave.  The emulation shows that
this alone sends waves 4-7 of the up tile 256-511 rows past each tile's first row, 1 MiB past the
end of X and W1 for the last tile row and column, while the role split of ffn_gemm_kernel keeps
every offset of every ticket inside its operand.
"""
import re
from dataclasses import dataclass
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
VARIANTS = ROOT / "ffn_optim_amd" / "csrc" / "ffn_variants.hpp"


@dataclass(frozen=True)
class Tile:
    """The TileCfg quantities the refill addressing uses (ffn_gemm.hpp, struct TileCfg)."""
    vid: int
    bm: int
    bn: int
    bk: int
    wgm: int
    wgn: int
    stages: int
    wgk: int = 1
    dmaw: int = 0
    prod: int = 0

    @property
    def nw(self):
        return self.wgm * self.wgn * self.wgk

    @property
    def dw(self):
        return self.prod if self.prod > 0 else (self.nw if self.dmaw == 0 else self.dmaw)

    @property
    def rowb(self):
        return self.bk * 2

    @property
    def rpb(self):
        return 1024 // self.rowb

    @property
    def a_blks(self):
        return self.bm * self.rowb // 1024

    @property
    def b_blks(self):
        return self.bn * self.rowb // 1024

    @property
    def a_pw(self):
        return self.a_blks // self.dw

    @property
    def b_pw(self):
        return self.b_blks // self.dw

    @property
    def loads(self):
        return self.a_pw + self.b_pw

    @property
    def stage_bytes(self):
        return (self.bm + self.bn) * self.rowb

    @property
    def k_iter_bytes(self):
        return self.bk * 2


def load_tiles():
    """Every X(id, BM, BN, BK, WGM, WGN, STAGES[, SYNCQ, DMAKS, WGK, DMAW, PROD, BDB]) row."""
    tiles = {}
    for args in re.findall(r"^\s*X\(([^)]*)\)", VARIANTS.read_text(), re.M):
        v = [int(a) for a in args.split(",")]
        extra = v[7:] + [-1, -1, 1, 0, 0, 0][len(v) - 7:]
        tiles[v[0]] = Tile(v[0], *v[1:7], wgk=extra[2], dmaw=extra[3], prod=extra[4])
    return tiles


TILES = load_tiles()


def issuing_waves(t, every_wave=False):
    """Waves that run the refill: ffn_gemm_kernel's dispatch (refill-only waves [0, PROD), or
    waves [0, DW)), or -- the removed single-launch kernel -- every wave of the workgroup."""
    waves = t.nw + t.prod
    return range(waves) if every_wave else range(t.dw)


def refill_blocks(t, wave):
    """(operand, block) of each of the LOADS DMA instructions the wave issues per stage."""
    out = []
    for d in range(t.loads):
        if d < t.a_pw:
            out.append(("a", wave * t.a_pw + d))
        else:
            out.append(("b", wave * t.b_pw + (d - t.a_pw)))
    return out


@pytest.mark.parametrize("vid", sorted(TILES))
def test_refill_fills_each_block_of_a_stage_once(vid):
    """ffn_gemm_kernel's issuing waves write every 1 KiB block of a stage exactly once, and only
    rows [0, BM) of A and [0, BN) of B: the per-wave block split is exact for every variant."""
    t = TILES[vid]
    assert t.a_blks % t.dw == 0 and t.b_blks % t.dw == 0
    seen = {}
    for w in issuing_waves(t):
        for op, blk in refill_blocks(t, w):
            seen[(op, blk)] = seen.get((op, blk), 0) + 1
            rows = t.bm if op == "a" else t.bn
            assert blk * t.rpb + t.rpb <= rows
            lds = (blk * 1024 if op == "a" else t.a_blks * 1024 + blk * 1024)
            assert lds + 1024 <= t.stage_bytes
    assert seen == {**{("a", b): 1 for b in range(t.a_blks)}, **{("b", b): 1 for b in range(t.b_blks)}}


def test_only_the_dmaw_tile_breaks_when_every_wave_refills():
    """With every wave issuing, the tiles whose refill is on a subset of their waves (DMAW, the
    eight-wave 256x256 tile) address blocks past the tile; the tiles whose waves all refill do
    not.  (Refill-only waves are numbered first, so the tile waves after them would too.)"""
    broken = set()
    for vid, t in TILES.items():
        for w in issuing_waves(t, every_wave=True):
            for op, blk in refill_blocks(t, w):
                if blk >= (t.a_blks if op == "a" else t.b_blks):
                    broken.add(vid)
    assert 12 in broken
    assert broken == {vid for vid, t in TILES.items() if t.dw < t.nw + t.prod}


# --- the removed single-launch kernel's schedule --------------------------------------------

def fused_tickets(tiles_m_up, tiles_n_up, tiles_m_down, tiles_n_down, ratio):
    """Tile coordinates of every ticket of every XCD queue: XCD x owns up row-blocks x, x + 8, ...
    and the down tiles of their rows; its queue hands out every up tile, then every down tile."""
    for x in range(8):
        rbs = list(range(x, tiles_m_up, 8))
        for rb in rbs:
            for tn in range(tiles_n_up):
                yield x, "up", rb, tn
        for rb in rbs:
            for dr in range(rb * ratio, min((rb + 1) * ratio, tiles_m_down)):
                for tn in range(tiles_n_down):
                    yield x, "down", dr, tn


def refill_span(t, tm, tn, k, m_rows, lda, n_rows, ldb, every_wave):
    """Largest byte offset (exclusive) of the SALU-addressed refill of tile (tm, tn) over all
    K-iterations of a K-deep reduction, for A and B, and the rows it reaches; the lane's
    16-byte chunk stays inside its row, so row r ends at (r * ld + k) * 2 bytes."""
    a_end = b_end = 0
    for w in issuing_waves(t, every_wave):
        for op, blk in refill_blocks(t, w):
            last_row = blk * t.rpb + t.rpb - 1
            if op == "a":
                a_end = max(a_end, ((tm * t.bm + last_row) * lda + k) * 2)
            else:
                b_end = max(b_end, ((tn * t.bn + last_row) * ldb + k) * 2)
    return a_end, b_end


@pytest.mark.parametrize("every_wave", [False, True])
def test_single_launch_schedule_of_the_faulting_run(every_wave):
    """Aligned mid-size FFN (X [4096, 1024], W1 [4096, 1024], W2 [1024, 4096], bf16), up on the
    eight-wave 256x256 tile (variant 12), down on the K-sliced eight-wave 128x128 tile
    (variant 13), 256 workgroups.  Every ticket of every XCD: with ffn_gemm_kernel's role split
    every refill stays inside X, W1, hidden and W2; with every wave refilling -- what the removed
    kernel did -- the up tiles of the last row and column read 1 MiB past X and W1."""
    up, dn = TILES[12], TILES[13]
    m, k, h, n = 4096, 1024, 4096, 1024
    tiles_m_up, tiles_n_up = m // up.bm, h // up.bn
    tiles_m_dn, tiles_n_dn = m // dn.bm, n // dn.bn
    ratio = up.bm // dn.bm
    sizes = {"x": m * k * 2, "w1": h * k * 2, "hidden": m * h * 2, "w2": n * h * 2}
    tickets = list(fused_tickets(tiles_m_up, tiles_n_up, tiles_m_dn, tiles_n_dn, ratio))
    # every tile of both GEMMs is handed out exactly once
    assert sorted((ph, a, b) for _, ph, a, b in tickets) == sorted(
        [("up", a, b) for a in range(tiles_m_up) for b in range(tiles_n_up)]
        + [("down", a, b) for a in range(tiles_m_dn) for b in range(tiles_n_dn)])
    past = []
    for x, phase, tm, tn in tickets:
        if phase == "up":
            a_end, b_end = refill_span(up, tm, tn, k, m, k, h, k, every_wave)
            ops = (("x", a_end), ("w1", b_end))
        else:
            a_end, b_end = refill_span(dn, tm, tn, h, m, h, n, h, every_wave)
            ops = (("hidden", a_end), ("w2", b_end))
        past += [(x, phase, tm, tn, name, end - sizes[name]) for name, end in ops if end > sizes[name]]
    if not every_wave:
        assert past == []
    else:
        assert past and {p[4] for p in past} == {"x", "w1"}
        assert max(p[5] for p in past) == 256 * k * 2   # 256 rows of 1024 bf16: 1 MiB
        # the last up tile row (row-block 15, XCD 7) and every tile of the last column
        assert {(p[0], p[2]) for p in past if p[4] == "x"} == {(7, 15)}
        assert {p[3] for p in past if p[4] == "w1"} == {tiles_n_up - 1}


FUSED_PAIRS = [tuple(int(v) for v in pair) for pair in re.findall(
    r"X\((\d+),\s*(\d+)\)", re.search(r"^#define FFN_FUSED_PAIRS\(X\)(.*)$", VARIANTS.read_text(), re.M).group(1))]


@pytest.mark.parametrize("pair,shape", [
    ((12, 21), (4096, 4096, 1024, 4096, 1024)),      # aligned mid-size: (m, mp, k, h, n)
    ((13, 19), (1005, 1024, 1008, 3008, 1024)),      # unaligned, padded buffers
    ((12, 17), (8192, 8192, 3072, 12288, 3072)),     # DiT-size
])
def test_single_launch_pairs_stay_inside_their_operands(pair, shape):
    """The compiled single-launch pairs (ffn_fused.hip) on the workloads they serve: both tiles
    have the same number of waves, the up tile's rows hold whole down tile rows, every XCD owns
    an up row block, every tile is handed out once, and with the kernels' role split every
    SALU-addressed refill of an interior tile (the others take the range-checked refill) stays
    inside its operand."""
    assert pair in FUSED_PAIRS
    up, dn = TILES[pair[0]], TILES[pair[1]]
    m, mp, k, h, n = shape
    assert up.nw + up.prod == dn.nw + dn.prod and up.bm % dn.bm == 0
    tiles_m_up, tiles_n_up = -(-m // up.bm), -(-h // up.bn)
    tiles_m_dn, tiles_n_dn = -(-m // dn.bm), -(-n // dn.bn)
    assert tiles_m_up >= 8
    tickets = list(fused_tickets(tiles_m_up, tiles_n_up, tiles_m_dn, tiles_n_dn, up.bm // dn.bm))
    assert sorted((ph, a, b) for _, ph, a, b in tickets) == sorted(
        [("up", a, b) for a in range(tiles_m_up) for b in range(tiles_n_up)]
        + [("down", a, b) for a in range(tiles_m_dn) for b in range(tiles_n_dn)])
    # a down tile's rows lie in an up row block of its own XCD
    for x, phase, tm, _ in tickets:
        if phase == "down":
            assert (tm * dn.bm // up.bm) % 8 == x
    sizes = {"x": mp * k * 2, "w1": h * k * 2, "hidden": mp * h * 2, "w2": n * h * 2}
    for x, phase, tm, tn in tickets:
        t, rows, cols, depth, a_name, b_name = ((up, m, h, k, "x", "w1") if phase == "up"
                                                else (dn, m, n, h, "hidden", "w2"))
        if (tm + 1) * t.bm > rows or (tn + 1) * t.bn > cols:
            continue   # edge tile: range-checked refill
        a_end, b_end = refill_span(t, tm, tn, depth, mp, depth, cols, depth, every_wave=False)
        assert a_end <= sizes[a_name] and b_end <= sizes[b_name], (phase, tm, tn)
