"""CPU emulation of the in-launch Stream-K finish (csrc/ffn_gemm.hpp, Engine::finish_piece).

Every piece of a split tile stores its FP32 partial and counts in on the tile's arrival counter
(one per tile and wave); the wave whose fetch-and-add returns pieces - 1 arrived last, resets the
counter and sums the pieces.  The emulation below follows finish_piece line by line -- the
keep / nth / set logic and the PC-wide loads -- and checks, for tiles of 2 to 6 pieces and every
arrival order, that the sum taken is the left fold of the pieces in ascending K order
(((p0 + p1) + p2) + ...), bit for bit on random FP32 partials, whichever piece arrives last.  The
one exception is the two-piece tile finished by its second piece, which adds p1 + p0: IEEE
addition is commutative, so that is bit-equal too.  The piece ranges themselves come from the
split schedule (sk_owner / sk_start, ops/kernel/ffn.py:653-665): consecutive workgroups own
consecutive K ranges, so ascending workgroup order is ascending K order.
"""
import itertools

import numpy as np
import pytest

from ffn_optim_amd import _lib


def finish_order(first, last, v, pc):
    """The additions finish_piece performs when workgroup v's wave arrives last: a list of
    (operation, piece) with operation 'own' (the piece in registers), 'set' (the first piece read
    replaces the registers) or 'add'."""
    keep = v == first or last - first == 1

    def nth(w0, k):
        return w0 + k + (1 if (keep and w0 <= v and w0 + k >= v) else 0)

    ops = [("own", v)] if keep else []
    set_ = not keep
    w = first
    while nth(w, 0) <= last:
        loaded = [nth(w, k) for k in range(pc) if nth(w, k) <= last]
        for k, piece in enumerate(loaded):
            ops.append(("set" if (set_ and k == 0) else "add", piece))
        set_ = False
        w = nth(w, pc - 1) + 1
    return ops


def fold(ops, partials):
    acc = None
    for op, piece in ops:
        acc = partials[piece] if op in ("own", "set") else np.float32(acc + partials[piece])
    return acc


@pytest.mark.parametrize("pieces", [2, 3, 4, 5, 6])
@pytest.mark.parametrize("pc", [1, 4])
def test_finish_sums_in_ascending_k_for_every_arrival_order(pieces, pc):
    rng = np.random.default_rng(pieces * 10 + pc)
    first = 3                      # the tile's first piece belongs to workgroup 3
    last = first + pieces - 1
    for order in itertools.permutations(range(first, last + 1)):
        counter, finisher = 0, None
        for v in order:            # arrivals: fetch-and-add on the tile's counter
            old, counter = counter, counter + 1
            if old == last - first:
                finisher, counter = v, 0
        assert finisher == order[-1] and counter == 0
        ops = finish_order(first, last, finisher, pc)
        used = [p for _, p in ops]
        assert sorted(used) == list(range(first, last + 1))          # every piece once
        if pieces == 2 and finisher == last:
            assert used == [last, first]                              # p1 + p0
        else:
            assert used == list(range(first, last + 1))               # ascending K
        assert ops[0][0] in ("own", "set") and all(op == "add" for op, _ in ops[1:])
        partials = {p: np.float32(x) for p, x in
                    zip(range(first, last + 1), rng.standard_normal(pieces).astype(np.float32) * 1e3)}
        want = partials[first]
        for p in range(first + 1, last + 1):
            want = np.float32(want + partials[p])
        assert fold(ops, partials).tobytes() == want.tobytes()


def _owner(x, q, r):
    """sk_owner: the workgroup owning split iteration x (q iterations each, one more for the
    first r)."""
    big = (q + 1) * r
    return x // (q + 1) if x < big else r + (x - big) // q


@pytest.mark.parametrize("shape", [(64, 5120, 13824, 5120, 16), (4096, 1024, 4096, 1024, 4096),
                                   (1024, 1008, 3008, 1024, 1005), (8192, 3072, 12288, 3072, 8192)])
def test_pieces_are_consecutive_workgroups_in_k_order(shape):
    """On the Stream-K plans of the decode, aligned mid-size, unaligned and DiT-size FFNs, the
    pieces of every split tile belong to consecutive workgroups first..last whose K ranges follow
    each other, and each fits the slots the plan reserves per workgroup."""
    mp, kp, hp, np_, m = shape
    plan = _lib.make_plan(mp, kp, hp, np_, _lib.BF16, "streamk", "erf", 256, m=m)
    kI, sk, G = plan.down_k_iters, plan.down_sk_tiles, plan.down_grid
    total = sk * kI
    q, r = total // G, total % G
    for s in range(sk):
        first, last = _owner(s * kI, q, r), _owner(s * kI + kI - 1, q, r)
        ranges = []
        for w in range(first, last + 1):
            start = w * q + min(w, r)
            end = (w + 1) * q + min(w + 1, r)
            lo, hi = max(start, s * kI), min(end, (s + 1) * kI)
            assert lo < hi
            ranges.append((lo, hi))
            assert s - start // kI < plan.down_slots_per_wg   # slot index of this piece
        assert ranges[0][0] == s * kI and ranges[-1][1] == (s + 1) * kI
        assert all(a[1] == b[0] for a, b in zip(ranges, ranges[1:]))
