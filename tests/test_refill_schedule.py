"""The LDS refill schedule of every compiled tile, replayed on the CPU.

The engine (ffn_optim_amd/csrc/ffn_gemm.hpp: Engine::prologue, mainloop, step, ksteps, slot)
interleaves, slot by slot, each wave's fragment reads of an LDS stage, the refill DMA of the
stages, the stage waits (s_waitcnt vmcnt) and the workgroup barriers.  This test follows that
code for one refilling wave -- every refilling wave runs the same slots with other blocks, and
every wave passes the same barriers -- over one unit and over two units in a row (the second
unit's DMA prologue goes out in the first unit's last k-step), and checks the two rules the
schedule must keep:

* read after refill: a read of a stage comes after a barrier, and before that barrier a wait
  has completed every load of the iteration the stage holds (loads complete in issue order);
* refill after read: a load into a stage comes after a barrier that follows the last read of
  the iteration the stage held before (the barrier helper waits for the wave's LDS reads).

The early refill (TileCfg's EARLY argument) is the case this guards most: part of an iteration's
refill goes out right after the stage barrier of the iteration two before, into the stage that
iteration read.  Planted mistakes (the early part into the other stage, or before the barrier,
or a first stage wait that counts the whole prologue as allowed in flight) must each break a
rule.

The tile parameters come from csrc/ffn_variants.hpp, the file the library is compiled from.
"""
from __future__ import annotations

import re
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parent.parent / "ffn_optim_amd" / "csrc"
NAMES = ("bm", "bn", "bk", "wgm", "wgn", "stages", "syncq", "dmaks", "wgk", "dmaw", "prod", "early", "mf")
DEFAULTS = dict(syncq=-1, dmaks=-1, wgk=1, dmaw=0, prod=0, early=0, mf=32)


def tiles() -> dict[int, dict]:
    """Every X(id, ...) row of FFN_VARIANTS, with TileCfg's defaults filled in."""
    text = (CSRC / "ffn_variants.hpp").read_text()
    body = text[text.index("#define FFN_VARIANTS(X)"):text.index("#define FFN_NUM_VARIANTS")]
    out = {}
    for args in re.findall(r"X\(([-\d,\s]+)\)", body):
        vals = [int(a) for a in args.split(",")]
        cfg = dict(DEFAULTS)
        cfg.update(zip(NAMES, vals[1:]))
        out[vals[0]] = derived(cfg)
    assert out and sorted(out) == list(range(len(out)))
    return out


def derived(c: dict) -> dict:
    """TileCfg's and Engine's compile-time constants (ffn_gemm.hpp)."""
    c = dict(c)
    nw = c["wgm"] * c["wgn"] * c["wgk"]
    mf = c["mf"]
    c["FM"], c["FN"] = c["bm"] // c["wgm"] // mf, c["bn"] // c["wgn"] // mf
    c["NM"] = c["FM"] * c["FN"]
    c["KS"] = c["bk"] // (512 // mf) // c["wgk"]
    c["SPLIT"] = mf == 16
    c["S"] = c["stages"]
    dw = c["prod"] if c["prod"] > 0 else (nw if c["dmaw"] == 0 else c["dmaw"])
    rowb = c["bk"] * 2
    a_blks, b_blks = c["bm"] * rowb // 1024, c["bn"] * rowb // 1024
    c["LOADS"] = a_blks // dw + b_blks // dw
    c["SYNC_Q"] = c["syncq"] if c["syncq"] >= 0 else (c["NM"] // 2 - 1 if c["SPLIT"] else c["FM"] - 1)
    c["PRO_Q"] = c["NM"] - 1 if c["SPLIT"] else c["SYNC_Q"]
    S, KS, NM = c["S"], c["KS"], c["NM"]
    c["DMA_ALL"] = S > 2 and c["dmaks"] * 16 == KS * (512 // mf)
    if S == 2:
        c["DMA_SLOTS"] = c["dmaks"] * NM * 16 // (512 // mf) if c["dmaks"] > 0 else KS // 2 * NM
    elif c["DMA_ALL"]:
        c["DMA_SLOTS"] = KS * NM
    else:
        c["DMA_SLOTS"] = (KS - 1) * NM + c["SYNC_Q"]
    before = ((KS - 1) * NM + c["SYNC_Q"]) * c["LOADS"] // c["DMA_SLOTS"] if c["DMA_ALL"] else c["LOADS"]
    c["STAGE_WAIT"] = c["LOADS"] * (S - 3) + before
    return c


class Wave:
    """Program order of one refilling wave: loads, LDS reads, waits and barriers."""

    def __init__(self):
        self.events = []   # ("load", stage, key, d) | ("read", stage, key) | ("wait", n) | ("barrier",)

    def load(self, stage, key, d):
        self.events.append(("load", stage, key, d))

    def read(self, stage, key):
        self.events.append(("read", stage, key))

    def wait(self, n):
        self.events.append(("wait", n))

    def barrier(self):
        self.events.append(("barrier",))


def run_units(c: dict, units: list[int], mutation: str | None = None) -> Wave:
    """The slot schedule of consecutive units of `units[i]` iterations each.  A key names an
    iteration as (unit, k); iterations past a unit still get (zero-fill) loads, as in the
    kernel."""
    S, KS, NM, FM, FN = c["S"], c["KS"], c["NM"], c["FM"], c["FN"]
    LOADS, EARLY, SYNC_Q, DMA_SLOTS = c["LOADS"], c["early"], c["SYNC_Q"], c["DMA_SLOTS"]
    w = Wave()

    def prologue(u):
        for s in range(S - 1):
            for d in range(LOADS):
                w.load(s, (u, s), d)
        for d in range(EARLY):
            w.load(S - 1, (u, S - 1), d)

    def kstep(u, it, cur, ksi, last, dstage):
        mode = 0 if ksi + 1 < KS else (2 if last else 1)
        nxt = (cur + 1) % S
        half = NM // 2 if NM // 2 > 0 else 1
        split, hs, fmh = c["SPLIT"], NM // 2, FM // 2
        # split order (16x16 blocks): the last slot of a k-step using each A / B fragment
        last_use = ([(i // fmh) * hs + (FN - 1) * fmh + i % fmh for i in range(FM)]
                    + [hs + j * fmh + fmh - 1 for j in range(FN)]) if split else []
        for q in range(NM):
            j, i = q // FM, q % FM
            # (the MFMA of slot q uses registers only)
            if mode == 0 and split:
                for lu in last_use:
                    if lu == q:
                        w.read(cur, (u, it))
            elif mode == 0:
                a0, a1 = q * FM // half, min((q + 1) * FM // half, FM)
                if q < half and a1 > a0:
                    w.read(cur, (u, it))
                if i == FM - 1:
                    w.read(cur, (u, it))
            else:
                if mode == 1 and q == SYNC_Q:
                    w.wait(0 if S == 2 else c["STAGE_WAIT"])
                    w.barrier()
                elif mode == 2 and q == c["PRO_Q"] and u + 1 < len(units):
                    w.barrier()
                    prologue(u + 1)
                if mode == 1 and q < SYNC_Q and split and mutation == "split_next_stage_before_barrier":
                    # the planted mistake: a fragment freed before the stage barrier read from the
                    # next stage at once
                    for lu in last_use:
                        if lu == q:
                            w.read(nxt, (u, it + 1))
                if mode == 1 and q >= SYNC_Q:
                    span, qq = NM - SYNC_Q, q - SYNC_Q
                    if split:
                        for lu in last_use:
                            if max(lu, SYNC_Q) == q and not (mutation == "split_next_stage_before_barrier"
                                                             and lu < SYNC_Q):
                                w.read(nxt, (u, it + 1))
                    else:
                        a0, a1 = qq * FM // span, (qq + 1) * FM // span
                        if a1 > a0:
                            w.read(nxt, (u, it + 1))
                        for jj in range(FN):
                            if max(jj * FM + FM - 1, SYNC_Q) == q:
                                w.read(nxt, (u, it + 1))
                    if EARLY and not last and mutation != "early_before_barrier":
                        e0, e1 = qq * EARLY // span, (qq + 1) * EARLY // span
                        stage = nxt if mutation == "early_into_next_stage" else cur
                        for d in range(e0, e1):
                            w.load(stage, (u, it + 2), d)
            g = ksi * NM + q
            if not last and g < DMA_SLOTS and (c["DMA_ALL"] or ksi + 1 < KS or q < SYNC_Q):
                t0 = EARLY + g * (LOADS - EARLY) // DMA_SLOTS
                t1 = EARLY + (g + 1) * (LOADS - EARLY) // DMA_SLOTS
                for d in range(t0, t1):
                    w.load(dstage, (u, it + S - 1), d)
            if mode == 1 and q == SYNC_Q - 1 and EARLY and mutation == "early_before_barrier":
                for d in range(EARLY):
                    w.load(cur, (u, it + 2), d)

    for u, n in enumerate(units):
        if u == 0:
            prologue(0)
        first = u == 0
        # the first stage wait lets the early part of iteration S-1 stay in flight; the planted
        # mistake confuses it with the whole prologue's count (Engine::PRO_LOADS)
        first_wait = LOADS * (S - 1) + EARLY if mutation == "first_wait_is_the_prologue_count" else LOADS * (S - 2) + EARLY
        w.wait(first_wait if first else 0)
        w.barrier()
        w.read(0, (u, 0))
        cur = 0
        for it in range(n - 1):
            dstage = S - 1 if cur == 0 else cur - 1
            for ksi in range(KS):
                kstep(u, it, cur, ksi, False, dstage)
            cur = (cur + 1) % S
        for ksi in range(KS):
            kstep(u, n - 1, cur, ksi, True, 0)
    return w


def violations(c: dict, w: Wave) -> list[str]:
    """Reads not covered by a wait + barrier over their iteration's loads, and loads into a stage
    not preceded by a barrier after the last read of the stage's previous iteration."""
    LOADS = c["LOADS"]
    bad = []
    outstanding = []        # loads issued and not yet waited for, in issue order
    done = set()            # (stage, key, d) completed
    covered = {}            # (stage, key) -> loads complete at the latest barrier
    issued = {}             # (stage, key) -> load indices issued
    complete_at_barrier = set()
    last_read = {}          # stage -> (key, event index)
    last_barrier = -1
    for idx, ev in enumerate(w.events):
        if ev[0] == "load":
            _, stage, key, d = ev
            issued.setdefault((stage, key), set()).add(d)
            prev = last_read.get(stage)
            if prev is not None and prev[0] != key and prev[1] > last_barrier:
                bad.append(f"event {idx}: load into stage {stage} for {key} before a barrier after "
                           f"the read of {prev[0]}")
            outstanding.append((stage, key, d))
        elif ev[0] == "wait":
            # s_waitcnt vmcnt(n): every load but the last n issued has completed
            k = max(0, len(outstanding) - ev[1])
            done.update(outstanding[:k])
            outstanding = outstanding[k:]
        elif ev[0] == "barrier":
            last_barrier = idx
            complete_at_barrier = set(done)
        else:
            _, stage, key = ev
            need = {(stage, key, d) for d in range(LOADS)}
            if not need <= complete_at_barrier:
                missing = sorted(d for (_, _, d) in need - complete_at_barrier)
                bad.append(f"event {idx}: read of stage {stage} ({key}) before loads {missing[:4]} "
                           f"were waited for ahead of a barrier")
            last_read[stage] = (key, idx)
    return bad


UNIT_SHAPES = [[1], [2], [3], [5], [8], [2, 3], [3, 1], [4, 4], [1, 2]]


@pytest.mark.parametrize("variant", sorted(tiles()))
def test_every_tile_keeps_the_refill_rules(variant):
    c = tiles()[variant]
    for units in UNIT_SHAPES:
        w = run_units(c, units)
        bad = violations(c, w)
        assert not bad, (variant, units, bad[:3])


def early_tiles():
    return [v for v, c in tiles().items() if c["early"]]


def test_some_tile_takes_the_early_refill():
    assert early_tiles(), "no compiled tile issues part of its refill early"


@pytest.mark.parametrize("mutation", ["early_into_next_stage", "early_before_barrier", "first_wait_is_the_prologue_count"])
def test_planted_mistakes_in_the_early_refill_are_caught(mutation):
    """Each mistake breaks a rule on every early-refill tile, for some unit shape."""
    for v in early_tiles():
        c = tiles()[v]
        assert any(violations(c, run_units(c, units, mutation)) for units in UNIT_SHAPES), (v, mutation)


def split_tiles():
    return [v for v, c in tiles().items() if c["SPLIT"]]


def test_planted_mistake_in_the_split_order_is_caught():
    """16x16 tiles read a fragment freed before the stage barrier only after it: reading the next
    stage at once breaks the read-after-refill rule."""
    assert split_tiles(), "no compiled tile takes 16x16x32 blocks"
    for v in split_tiles():
        c = tiles()[v]
        assert any(violations(c, run_units(c, units, "split_next_stage_before_barrier"))
                   for units in UNIT_SHAPES), v
