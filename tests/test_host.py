"""CPU tests of the host side: input contract, selection, planning, Stream-K schedule, C ABI.

Restates the reference's CPU tests (validation/test_ffn.py InputTests :24-74 and
test_selection :172-183) against this package, plus checks of the native plan.
"""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from ffn_optim_amd import _lib
from ffn_optim_amd.cases import (BENCH_CASES, V1_CASES, case_problem, load_cases,
                                 make_inputs)
from ffn_optim_amd.host.dispatch import (DependencyUnavailable, NotApplicable, Selection,
                                         verify_dependency)
from ffn_optim_amd.host.inputs import prepare_storage, problem_from_shapes, validate_tensors
from ffn_optim_amd.host.tiling import make_plan
from oracle.reference import compare, ffn_torch

REPO = Path(__file__).resolve().parents[1]


def test_ranks_and_padding():
    """validation/test_ffn.py:31-48: padded storage gives the unpadded result, shape restored."""
    for dtype in (torch.float16, torch.bfloat16):
        for rank in range(2, 9):
            shape = (1,) * (rank - 2) + (3, 17)
            x = torch.randn((*shape[:-1], 34)).to(dtype)[..., ::2]
            w1 = torch.randn(19, 34).to(dtype)[:, ::2]
            w2 = torch.randn(23, 38).to(dtype)[:, ::2]
            p = validate_tensors(x, w1, w2)
            plan = make_plan(p)
            (xp, a, b, hidden, out, ws), layout, x_rows = prepare_storage(x, w1, w2, plan)
            assert layout == (p.k if p.k % 8 == 0 else plan.kp, p.h, p.n, plan.kp, plan.kp, plan.hp)
            assert xp.shape == (plan.mp, plan.kp) and a.shape == (plan.hp, plan.kp)
            assert b.shape == (plan.np, plan.hp) and hidden.shape == (plan.mp, plan.hp)
            assert out.shape == (plan.mp, plan.np) and ws.dtype == torch.float32
            assert int(xp[p.m:].abs().sum()) == 0 and int(xp[:, p.k:].abs().sum()) == 0
            got = ffn_torch(xp, a, b, staged=True)[:p.m, :p.n].view(p.output_shape)
            ref = ffn_torch(x, w1, w2, staged=True)
            assert compare(got, ref)["passed"]
            assert got.shape == (*shape[:-1], 23)


def test_invalid_shapes():
    """validation/test_ffn.py:50-59."""
    p = problem_from_shapes
    for args in [([3], [4, 3], [3, 4]), ([0, 3], [4, 3], [3, 4]),
                 ([2, 3], [4, 2], [3, 4]), ([1] * 9, [4, 1], [3, 4]),
                 ([True, 3], [4, 3], [3, 4]), ([2, 65536], [4, 65536], [3, 4])]:
        with pytest.raises(ValueError):
            p(*args)
    for kwargs in ({"dtype": "float32"}, {"layout": "canonical"}):
        with pytest.raises(ValueError):
            p([2, 3], [4, 3], [3, 4], **kwargs)


def test_no_device_fallback():
    """validation/test_ffn.py:61-65: CPU tensors are refused, never computed on the host."""
    from ffn_optim_amd import ffn
    with pytest.raises(ValueError, match="requires ROCm GPU"):
        ffn(torch.zeros(2, 3).half(), torch.zeros(4, 3).half(), torch.zeros(3, 4).half())


def test_invalid_tensors():
    """validation/test_ffn.py:67-74."""
    x, a, b = torch.zeros(2, 3).half(), torch.zeros(4, 3).half(), torch.zeros(3, 4).half()
    with pytest.raises(ValueError):
        validate_tensors(x, a.float(), b)
    with pytest.raises(ValueError):
        validate_tensors(x.requires_grad_(), a, b)
    with pytest.raises(TypeError):
        validate_tensors(x.detach().numpy(), a, b)


def test_selection():
    """validation/test_ffn.py:172-183 on this plan: full loads unavailable, Stream-K needs a
    remainder tile for its block_num."""
    for kind in ("full_load_a", "full_load_b"):
        with pytest.raises(DependencyUnavailable):
            Selection(down_impl=kind).require_available()
        with pytest.raises(DependencyUnavailable):
            make_plan(problem_from_shapes([64, 128], [256, 128], [64, 256]), Selection(down_impl=kind))
    with pytest.raises(ValueError):
        Selection(up_impl="streamk")
    with pytest.raises(ValueError):
        Selection(down_impl="splitk")
    p = problem_from_shapes([64, 128], [256, 128], [64, 256])
    plan = make_plan(p, Selection(down_impl="streamk"), 8)
    assert plan.workspace_bytes == plan.native.workspace_bytes > 0
    assert plan.schedule()["down_sk_tiles"] >= 1
    with pytest.raises(NotApplicable):
        make_plan(p, Selection(down_impl="streamk"), 1)
    with pytest.raises(NotApplicable):   # H spans a single K iteration of a 64-deep tile
        make_plan(problem_from_shapes([64, 128], [64, 128], [64, 64]), Selection(down_impl="streamk"),
                  8, down_variant=4)
    for bad in (0, 65536, 8.0, True):
        with pytest.raises(ValueError):
            make_plan(p, Selection(), bad)
    assert make_plan(p, Selection(), 8).workspace_shape == (1, 1)


def test_benchmark_cases_plan_for_both_down_impls():
    """Every measured workload is plannable for Basic and Stream-K at 256 workgroups."""
    for case in load_cases(BENCH_CASES):
        p = case_problem(case)
        for down in ("basic", "streamk"):
            plan = make_plan(p, Selection(down_impl=down), 256)
            assert plan.mp % 64 == 0 and plan.hp % 64 == 0 and plan.np % 64 == 0 and plan.kp % 16 == 0
            assert plan.up.bm * plan.up.bn > 0


def _sk_start(v, q, r):
    return v * q + min(v, r)


@pytest.mark.parametrize("G", [1, 7, 8, 37, 256])
def test_streamk_schedule_exact_once_and_slots(G):
    """The split schedule the kernel follows covers every (tile, K-iteration) exactly once and
    never needs more partial slots per workgroup than the plan reserves (brute force)."""
    for (mp, hp, np_) in [(64, 128, 64), (320, 1024, 448), (4096, 4096, 1024), (64, 13824, 5120),
                          (8192, 12288, 3072), (1024, 3008, 1024)]:
        for variant in range(_lib.load().ffn_mi355x_num_variants()):
            try:
                n = _lib.make_plan(mp, 64, hp, np_, _lib.BF16, "streamk", "erf", G, 0, variant)
            except ValueError:
                continue
            kI, dp, sk = n.down_k_iters, n.down_dp_tiles, n.down_sk_tiles
            Gs = n.down_grid      # block_num, or fewer workgroups that cut every tile evenly
            # every tile split into at most four pieces, equal ones where the iterations allow
            assert Gs <= G and (Gs == G or (n.down_tiles < G and Gs % n.down_tiles == 0
                                            and 2 <= Gs // n.down_tiles <= 4))
            assert dp + sk == n.down_tiles and sk == n.down_tiles % Gs and sk > 0
            total = sk * kI
            q, r = total // Gs, total % Gs
            seen = [[0] * kI for _ in range(sk)]
            for v in range(Gs):
                a, b = _sk_start(v, q, r), _sk_start(v + 1, q, r)
                tiles = {it // kI for it in range(a, b)}
                assert len(tiles) <= n.down_slots_per_wg
                for it in range(a, b):
                    seen[it // kI][it % kI] += 1
            assert all(c == 1 for row in seen for c in row)
            # the fixed region of arrival counters (one per split tile and wave), then the slots
            counters = _lib.workspace_counter_bytes(n)
            assert counters == 64 << 10 and sk * _lib.variants()[variant]["waves"] * 4 <= counters
            assert n.workspace_bytes == counters + Gs * n.down_slots_per_wg * n.down_bm * n.down_bn * 4


def test_tiles_report_their_mfma_edge():
    """Variants 22-25 take 16x16x32 MFMAs, every other tile 32x32x16; the query refuses an
    out-of-range variant."""
    infos = _lib.variants()
    assert {v["variant"] for v in infos if v["mfma_edge"] == 16} == {22, 23, 24, 25}
    assert all(v["mfma_edge"] == 32 for v in infos if v["variant"] not in (22, 23, 24, 25))
    with pytest.raises(ValueError):
        _lib.check(_lib.load().ffn_mi355x_variant_mfma_edge(len(infos)))
    with pytest.raises(ValueError):
        _lib.check(_lib.load().ffn_mi355x_variant_mfma_edge(-1))


def test_refill_wave_tiles_report_their_waves():
    """Tiles whose LDS refill is issued by waves of their own report them and count them in
    their waves; they plan like every other tile (whole, Stream-K and split up GEMMs), and the
    query refuses an out-of-range variant."""
    infos = _lib.variants()
    refill = [v for v in infos if v["refill_waves"] > 0]
    assert {v["variant"] for v in refill} == {17, 18, 19, 20, 21, 23, 24}
    for v in refill:
        assert v["waves"] > v["refill_waves"] > 0
        # decode down: 16 rows, 5120 wide, 13824 deep -- every tile count leaves a remainder
        plan = _lib.make_plan(64, 5120, 13824, 5120, _lib.BF16, "streamk", "erf", 256, 8, v["variant"], m=16)
        assert plan.down_variant == v["variant"] and plan.down_sk_tiles > 0
    assert all(v["refill_waves"] == 0 for v in infos if v not in refill)
    with pytest.raises(ValueError):
        _lib.check(_lib.load().ffn_mi355x_variant_refill_waves(len(infos)))


@pytest.mark.parametrize("G", [8, 37, 256])
def test_split_up_schedule_covers_once_and_shares_every_tile(G):
    """A split up GEMM (tiles filling at most half the grid, 16 or more K-iterations) covers
    every (tile, K-iteration) exactly once, shares every tile between two or more workgroups
    (its last piece applies the GELU), and its slots fit the workspace (brute force).
    Other up GEMMs keep one workgroup per tile."""
    lib = _lib.load()
    split_seen = 0
    for (mp, kp, hp) in [(64, 5120, 1728), (64, 1024, 4096), (320, 1008, 448), (128, 256, 1024),
                         (4096, 1024, 4096), (64, 5120, 13824)]:
        for variant in range(lib.ffn_mi355x_num_variants()):
            n = _lib.make_plan(mp, kp, hp, 64, _lib.BF16, "basic", "erf", G, variant, -1)
            kI, tiles = n.up_k_iters, n.up_tiles
            assert kI == -(-kp // n.up_bk)
            if n.up_sk_tiles == 0:
                assert tiles * 2 > G or kI < 16
                assert n.up_grid == min(tiles, G)
                continue
            split_seen += 1
            assert n.up_sk_tiles == tiles and tiles * 2 <= G and kI >= 16
            Gs = n.up_grid
            assert tiles < Gs <= G
            q, r = divmod(tiles * kI, Gs)
            seen = [[0] * kI for _ in range(tiles)]
            owners = [set() for _ in range(tiles)]
            for v in range(Gs):
                a, b = _sk_start(v, q, r), _sk_start(v + 1, q, r)
                assert len({it // kI for it in range(a, b)}) <= n.up_slots_per_wg
                for it in range(a, b):
                    seen[it // kI][it % kI] += 1
                    owners[it // kI].add(v)
            assert all(c == 1 for row in seen for c in row)
            assert all(len(o) >= 2 for o in owners)
            assert n.workspace_bytes >= (_lib.workspace_counter_bytes(n)
                                         + Gs * n.up_slots_per_wg * n.up_bm * n.up_bn * 4)
    assert split_seen > 0


def test_split_up_without_workspace_is_refused():
    """A plan that splits its up GEMM needs the workspace: ffn_mi355x_up and ffn_mi355x_run
    refuse a NULL ws before touching any buffer (no device call is made)."""
    lib = _lib.load()
    plan = _lib.make_plan(64, 5120, 1728, 5120, _lib.BF16, "basic", "erf", 256, m=16)
    assert plan.up_sk_tiles > 0 and plan.workspace_bytes > 0
    fake = 1 << 40                       # aligned, never dereferenced
    rc = lib.ffn_mi355x_up(ctypes.byref(plan), fake, fake, fake, None, None)
    assert rc == _lib.EINVAL and "workspace" in _lib.last_error()
    rc = lib.ffn_mi355x_run(ctypes.byref(plan), fake, fake, fake, fake, fake, None, None)
    assert rc == _lib.EINVAL and "workspace" in _lib.last_error()


def test_split_up_is_planned_for_the_decode_shard_only():
    """Of the measured workloads only the decode shard (16 x 5120 -> 1728: 27 tiles of 64x64)
    splits its up GEMM; its Basic plan then carries a workspace for the split."""
    from ffn_optim_amd.cases import SHARD_CASES
    for path in (BENCH_CASES, SHARD_CASES):
        for case in load_cases(path):
            p = case_problem(case)
            for down in ("basic", "streamk"):
                plan = make_plan(p, Selection(down_impl=down), 256)
                split = plan.native.up_sk_tiles > 0
                assert split == (case["case_id"] == "c4_tp8_shard_bf16"), (case["case_id"], down)
                if split:
                    assert plan.workspace_bytes >= plan.native.workspace_bytes > 0
                    assert plan.schedule()["up_sk_tiles"] == plan.native.up_tiles


def test_c_abi_exports_every_declared_symbol():
    header = (REPO / "include" / "ffn_mi355x.h").read_text()
    names = set(re.findall(r"^(?:int|const char\*)\s+(ffn_mi355x_\w+)\s*\(", header, re.M))
    assert len(names) >= 10
    lib = _lib.load()
    for name in names:
        assert hasattr(lib, name), name
    assert lib.ffn_mi355x_version().decode().startswith("ffn_mi355x gfx950")
    assert verify_dependency()["version"].startswith("ffn_mi355x gfx950")


def test_c_abi_error_codes_without_gpu():
    """Host-only entry points: argument errors map onto the reference's exception types."""
    with pytest.raises(ValueError, match="multiples of 64"):
        _lib.make_plan(100, 64, 64, 64, _lib.BF16, "basic", "erf", 8)
    with pytest.raises(DependencyUnavailable):
        _lib.make_plan(64, 64, 64, 64, _lib.BF16, "full_load_b", "erf", 8)
    with pytest.raises(ValueError, match="block_num"):
        _lib.make_plan(64, 64, 64, 64, _lib.BF16, "basic", "erf", 0)
    lib = _lib.load()
    rc = lib.ffn_mi355x_up(None, None, None, None, None, None)
    assert rc == _lib.EINVAL and "invalid plan" in _lib.last_error()
    info = _lib.variants()
    assert all(v["lds_bytes"] <= 160 * 1024 and v["waves"] >= 1 for v in info)


def test_make_inputs_contract():
    """common/cases.py:34-50: deterministic, scaled by fan-in, stride-2 and transposed views."""
    for case in load_cases(BENCH_CASES)[:1] + load_cases(V1_CASES):
        x, w1, w2 = make_inputs(case)
        x2, _, _ = make_inputs(case)
        assert torch.equal(x, x2)
        p = case_problem(case)
        assert tuple(x.shape) == p.input_shape and w1.shape == (p.h, p.k) and w2.shape == (p.n, p.h)
        if case.get("noncontiguous"):
            assert x.stride()[-1] == 2 and w1.stride()[-1] == 2
    case = load_cases(BENCH_CASES)[0]
    x, w1, w2 = make_inputs(case)
    assert abs(x.float().std().item() - 1.0) < 0.02
    assert abs(w1.float().std().item() * 256 ** 0.5 - 1.0) < 0.02
    assert abs(w2.float().std().item() * 1024 ** 0.5 - 1.0) < 0.02
    t = dict(load_cases(BENCH_CASES)[2], shape=[3, 5, 7, 8], weight1_shape=[9, 8],
             weight2_shape=[4, 9])
    xt, _, _ = make_inputs(t)
    xc, _, _ = make_inputs(dict(t, x_view=None))
    assert torch.equal(xt, xc) and not xt.is_contiguous() and xt.stride() == (280, 8, 40, 1)


def test_case_schema_rejects_bad_files(tmp_path):
    bad = tmp_path / "c.json"
    for text in ('{"schema_version": 2, "cases": []}', '{"schema_version": 1, "cases": []}',
                 '{"schema_version": 1, "cases": [{"case_id": "a", "shape": [2, 3], '
                 '"weight1_shape": [4, 3], "weight2_shape": [3, 4], "dtype": "float16", "seed": 1.5}]}'):
        bad.write_text(text)
        with pytest.raises(ValueError):
            load_cases(bad)


def test_operands_used_in_place_only_when_asked():
    import torch
    from ffn_optim_amd.host.dispatch import Selection
    from ffn_optim_amd.host.inputs import operands_aligned, prepare_storage, problem_from_shapes
    from ffn_optim_amd.host.tiling import make_plan
    g = torch.Generator().manual_seed(0)
    # aligned K/H/N, ragged M (m=100): X is used as [m, k] in place
    x = torch.randn(4, 25, 128, generator=g).half()
    w1, w2 = torch.randn(256, 128, generator=g).half(), torch.randn(64, 256, generator=g).half()
    plan = make_plan(problem_from_shapes(x.shape, w1.shape, w2.shape, "float16"), Selection(), 8)
    assert operands_aligned(x, w1, w2, plan)
    (xs, w1s, w2s, hid, out, ws), layout, x_rows = prepare_storage(x, w1, w2, plan, alias_aligned=True)
    assert xs.data_ptr() == x.data_ptr() and xs.shape == (100, 128)
    assert w1s is w1 and w2s is w2 and layout == (128, 256, 64, 128, 128, 256)
    assert hid.shape == (128, 256) and out.shape == (128, 64)
    # without the request the storage is a padded snapshot
    (xs, w1s, _, _, _, _), layout, x_rows = prepare_storage(x, w1, w2, plan)
    assert xs.data_ptr() != x.data_ptr() and xs.shape == (128, 128)
    assert torch.equal(xs[:100], x.view(100, 128)) and not xs[100:].any()
    assert layout == (128, 256, 64, plan.kp, plan.kp, plan.hp)
    # widths below the padded extents but whole 16-byte rows: still in place, unpadded
    x2 = torch.randn(37, 120, generator=g).half()
    w12, w22 = torch.randn(200, 120, generator=g).half(), torch.randn(72, 200, generator=g).half()
    p2 = make_plan(problem_from_shapes(x2.shape, w12.shape, w22.shape, "float16"), Selection(), 8)
    assert not operands_aligned(x2, w12, w22, p2)
    (xs, w1s, w2s, _, _, _), layout, _ = prepare_storage(x2, w12, w22, p2, alias_aligned=True)
    assert xs.data_ptr() == x2.data_ptr() and w1s is w12 and w2s is w22
    assert layout == (120, 200, 72, 120, 120, 200)
    # H not a multiple of 8: W2 is copied into [np, hp]; W1 [h, k] stays in place
    w13, w23 = torch.randn(201, 120, generator=g).half(), torch.randn(72, 201, generator=g).half()
    p3 = make_plan(problem_from_shapes(x2.shape, w13.shape, w23.shape, "float16"), Selection(), 8)
    (xs, w1s, w2s, _, _, _), layout, _ = prepare_storage(x2, w13, w23, p3, alias_aligned=True)
    assert w1s is w13 and w2s.shape == (p3.np, p3.hp) and not w2s[:, 201:].any()
    assert layout == (120, 201, 72, 120, 120, p3.hp)
    # K not a multiple of 8, or K not contiguous: copied and padded
    for xx, ww1 in ((torch.randn(100, 100, generator=g).half(), torch.randn(256, 100, generator=g).half()),
                    (torch.randn(128, 100, generator=g).half().t(), w1)):
        p = make_plan(problem_from_shapes(xx.shape, ww1.shape, w2.shape, "float16"), Selection(), 8)
        (xs, w1s, _, _, _, _), layout, x_rows = prepare_storage(xx, ww1, w2, p, alias_aligned=True)
        assert xs.data_ptr() != xx.data_ptr() and xs.shape == (p.mp, p.kp) and x_rows is None
        assert layout[3] == p.kp and (layout[0] == p.kp or xx.shape[-1] % 8 == 0)
    # a permuted X [25, 4, 128] of a [4, 25, 128] tensor: read in place as a row grid
    xt = x.transpose(0, 1)
    p = make_plan(problem_from_shapes(xt.shape, w1.shape, w2.shape, "float16"), Selection(), 8)
    (xs, _, _, _, _, _), layout, x_rows = prepare_storage(xt, w1, w2, p, alias_aligned=True)
    assert xs is xt and layout[3] == 128 and x_rows == (25, 4, 0, 128, 3200)
    # the same permuted X without the request: a padded snapshot
    (xs, _, _, _, _, _), layout, x_rows = prepare_storage(xt, w1, w2, p)
    assert xs.shape == (p.mp, p.kp) and x_rows is None and torch.equal(xs[:100], xt.reshape(100, 128))


def _rows_of(x, grid):
    """Gather the rows of X that a row_grid result addresses (the kernels' row addressing, on
    the CPU): row r of the [m / (d1*d2), d1, d2] grid at element i0*s0 + i1*s1 + i2*s2."""
    k = x.shape[-1]
    flat = torch.as_strided(x, (x.untyped_storage().nbytes() // x.element_size(),), (1,), 0)
    base = x.storage_offset()
    m = x.numel() // k
    if grid[0] == "pitch":
        starts = [base + r * grid[1] for r in range(m)]
    else:
        d1, d2, s0, s1, s2 = grid[1]
        starts = [base + (r // (d1 * d2)) * s0 + (r // d2 % d1) * s1 + (r % d2) * s2 for r in range(m)]
    return torch.stack([flat[s:s + k] for s in starts])


def test_row_grid_addresses_every_row():
    """row_grid: the rows it addresses are X.reshape(m, k) row for row, for contiguous, sliced,
    permuted and broadcast views; views it cannot address are refused (None)."""
    from ffn_optim_amd.host.inputs import row_grid
    base = torch.arange(2 * 3 * 5 * 7 * 64, dtype=torch.float32).half().view(2, 3, 5, 7, 64)
    views = {
        "contiguous": base.reshape(210, 64),
        "rank5": base,
        "sliced K": base.reshape(210, 64)[:, :32],
        "permuted": base.permute(1, 0, 2, 3, 4),
        "three groups": base.reshape(6, 5, 7, 64).permute(1, 0, 2, 3),
        "canonical": base.reshape(6, 35, 64).transpose(0, 1),
        "size-1 dims": base[:1, :1].permute(1, 0, 2, 3, 4),
        "row step": base.reshape(210, 64)[::2],
        "broadcast rows": base[0, 0, 0, :1].expand(9, 64),
    }
    want = {"contiguous": "pitch", "rank5": "pitch", "sliced K": "pitch", "permuted": "grid",
            "three groups": "grid", "canonical": "grid", "size-1 dims": "pitch",
            "row step": "pitch", "broadcast rows": "grid"}
    for name, v in views.items():
        grid = row_grid(v, v.shape[-1])
        assert grid is not None and grid[0] == want[name], (name, grid)
        assert torch.equal(_rows_of(v, grid), v.reshape(-1, v.shape[-1])), name
    refused = {
        "K strided": base.reshape(210, 64)[:, ::2],
        "K not a multiple of 8": base.reshape(210, 64)[:, :36],
        "four groups": base.permute(3, 2, 1, 0, 4),
        "off 16 bytes": base.reshape(210, 64)[:, 4:36],
        "K transposed": base.reshape(210, 64).t(),
    }
    for name, v in refused.items():
        assert row_grid(v, v.shape[-1]) is None, name


def test_row_grid_copies_rows_past_the_largest_pitch():
    """A column slice of rows wider than the library's largest pitch is copied (None), not
    handed to set_operands, which would refuse it; at the largest pitch it is read in place.
    The Python bound is the header's FFN_MI355X_MAX_PITCH, and the library enforces it."""
    from ffn_optim_amd.host.inputs import row_grid
    header = (Path(__file__).resolve().parent.parent / "include" / "ffn_mi355x.h").read_text()
    assert int(re.search(r"#define FFN_MI355X_MAX_PITCH (\d+)", header).group(1)) == _lib.MAX_PITCH
    for width, want in ((_lib.MAX_PITCH, ("pitch", _lib.MAX_PITCH)), (_lib.MAX_PITCH + 16, None)):
        base = torch.empty((2, width), dtype=torch.bfloat16)
        assert row_grid(base[:, :1024], 1024) == want
    plan = _lib.make_plan(64, 1024, 1024, 1024, _lib.BF16, "basic", "erf", 256, m=2)
    _lib.set_operands(plan, 1024, 1024, 1024, _lib.MAX_PITCH, 1024, 1024)
    with pytest.raises(ValueError):
        _lib.set_operands(plan, 1024, 1024, 1024, _lib.MAX_PITCH + 8, 1024, 1024)


def test_set_x_rows_validates_grid():
    """ffn_mi355x_set_x_rows accepts a grid that tiles m with 16-byte strides, keeps it through
    set_operands, and rejects the rest without touching the plan."""
    from ffn_optim_amd import _lib
    plan = _lib.make_plan(1024, 1008, 1024, 1024, _lib.FP16, "basic", "erf", 256, m=1005)
    _lib.set_operands(plan, 1000, 1024, 1024, 1000, 1000, 1024)
    _lib.set_x_rows(plan, 5, 67, 335000, 1000, 5000)
    assert (plan.x_d1, plan.x_d2, plan.x_s0, plan.x_s1, plan.x_s2) == (5, 67, 335000, 1000, 5000)
    _lib.set_operands(plan, 1000, 1024, 1024, 1000, 1000, 1024)
    assert (plan.x_d1, plan.x_d2) == (5, 67)
    for bad in ((4, 67, 335000, 1000, 5000),       # d1*d2 does not divide m
                (5, 67, 335000, 1000, 5004),       # stride not a multiple of 8
                (5, 67, -8, 1000, 5000),           # negative stride
                (5, 0, 335000, 1000, 5000),        # empty dim
                (5, 67, 2 ** 29, 1000, 5000)):     # rows spread over 2^31 bytes
        with pytest.raises(ValueError):
            _lib.set_x_rows(plan, *bad)
        assert (plan.x_d1, plan.x_d2, plan.x_s2) == (5, 67, 5000)
    _lib.set_x_rows(plan, 0, 0, 0, 0, 0)
    assert (plan.x_d1, plan.x_d2, plan.x_s0) == (0, 0, 0)


def test_set_operands_validates_layout():
    """ffn_mi355x_set_operands accepts logical widths with 16-byte rows and rejects the rest
    without touching the plan."""
    from ffn_optim_amd import _lib
    plan = _lib.make_plan(1024, 1008, 3008, 1024, _lib.FP16, "basic", "erf", 256, m=1005)
    assert (plan.k, plan.h, plan.n, plan.ldx, plan.ldw1, plan.ldw2) == (1008, 3008, 1024, 1008, 1008, 3008)
    _lib.set_operands(plan, 1000, 3001, 999, 1000, 1000, 3008)
    assert (plan.k, plan.h, plan.n, plan.ldx, plan.ldw1, plan.ldw2) == (1000, 3001, 999, 1000, 1000, 3008)
    for bad in ((1004, 3001, 999, 1008, 1008, 3008),   # K neither a multiple of 8 nor kp
                (1000, 3001, 999, 996, 1000, 3008),    # pitch below K
                (1000, 3001, 999, 1004, 1000, 3008),   # pitch not a multiple of 8
                (1000, 3001, 999, 1000, 1000, 3001),   # H not a multiple of 8 and W2 short of hp
                (1000, 3009, 999, 1000, 1000, 3016),   # H above hp
                (1000, 3000, 1025, 1000, 1000, 3000)): # N above np
        with pytest.raises(ValueError):
            _lib.set_operands(plan, *bad)
        assert (plan.k, plan.h, plan.n) == (1000, 3001, 999)


def _k_sliced_variants():
    """Variants with waves along K: the tenth field (WGK) of their row in ffn_variants.hpp."""
    text = (REPO / "ffn_optim_amd" / "csrc" / "ffn_variants.hpp").read_text()
    out = set()
    for m in re.finditer(r"^\s*X\(([^)]*)\)", text, re.M):
        fields = [int(f) for f in m.group(1).split(",")]
        if len(fields) >= 10 and fields[9] > 1:
            out.add(fields[0])
    return out


def test_k_sliced_variants_plan_for_basic_and_streamk():
    """The K-sliced tiles (two waves along K) report two, four or eight tile waves (plus their
    refill-only waves, if any), are planned for the up GEMM and the Basic down, and have a
    Stream-K form (the slices are summed before a split piece writes its partial)."""
    from ffn_optim_amd import _lib
    ids = _k_sliced_variants()
    assert {10, 11, 13, 14, 15, 16, 18, 19, 20, 21, 24} == ids
    sliced = [v for v in _lib.variants() if v["variant"] in ids]
    for v in sliced:
        assert v["waves"] - v["refill_waves"] in (2, 4, 8) and v["lds_bytes"] <= 160 * 1024
        plan = _lib.make_plan(4096, 1024, 4096, 1024, _lib.BF16, "basic", "erf", 256,
                              v["variant"], v["variant"])
        assert (plan.up_variant, plan.down_variant) == (v["variant"], v["variant"])
        assert plan.workspace_bytes == 0
        # decode down: 16 rows, 5120 wide, 13824 deep -- every tile count leaves a remainder
        plan = _lib.make_plan(64, 5120, 13824, 5120, _lib.BF16, "streamk", "erf", 256, 8, v["variant"], m=16)
        assert plan.down_variant == v["variant"] and plan.down_sk_tiles > 0 and plan.workspace_bytes > 0


def test_run_rejects_a_plan_whose_launch_fields_were_changed():
    """ffn_mi355x_run / _up / _down refuse a plan whose grids, tile counts, Stream-K split,
    workspace size or layout no longer match the stamp make_plan / set_operands wrote (no
    launch is made, so this runs without a GPU)."""
    import ctypes
    from ffn_optim_amd import _lib
    lib = _lib.load()
    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(6)]  # aligned, never dereferenced
    for down in ("basic", "streamk"):
        for field, delta in (("up_grid", 1), ("down_grid", -1), ("down_slots_per_wg", -1),
                             ("workspace_bytes", -256), ("down_sk_tiles", 1), ("up_bm", 64)):
            plan = _lib.make_plan(1024, 1008, 3008, 1024, _lib.FP16, down, "erf", 256)
            if down == "basic" and field in ("down_slots_per_wg", "workspace_bytes", "down_sk_tiles"):
                continue
            setattr(plan, field, getattr(plan, field) + delta)
            rc = lib.ffn_mi355x_run(ctypes.byref(plan), *fake, None)
            assert rc == -1 and "invalid plan" in lib.ffn_mi355x_last_error().decode(), (down, field)
            # nor does set_operands re-stamp a changed plan
            rc = lib.ffn_mi355x_set_operands(ctypes.byref(plan), 1008, 3008, 1024, 1008, 1008, 3008)
            assert rc == -1 and "invalid plan" in lib.ffn_mi355x_last_error().decode(), (down, field)
    # the layout fields are covered too: a pitch changed behind set_operands' back
    plan = _lib.make_plan(1024, 1008, 3008, 1024, _lib.FP16, "basic", "erf", 256)
    plan.ldx += 8
    assert lib.ffn_mi355x_run(ctypes.byref(plan), *fake, None) == -1


def test_operand_pitches_are_bounded():
    """Row pitches up to 4,000,000 elements keep a tile's 32-bit buffer offsets below the
    2^31 zero-fill marker; a larger pitch is refused (EINVAL) instead of reading wrong rows."""
    from ffn_optim_amd import _lib
    plan = _lib.make_plan(1024, 1024, 1024, 1024, _lib.BF16, "basic", "erf", 256)
    _lib.set_operands(plan, 1024, 1024, 1024, 4_000_000, 1024, 1024)
    for pitches in ((4_000_008, 1024, 1024), (1024, 4_000_008, 1024), (1024, 1024, 4_000_008)):
        plan = _lib.make_plan(1024, 1024, 1024, 1024, _lib.BF16, "basic", "erf", 256)
        with pytest.raises(ValueError, match="at most 4000000"):
            _lib.set_operands(plan, 1024, 1024, 1024, *pitches)


def test_streamk_grid_cuts_tiles_evenly_when_it_keeps_most_workgroups():
    """Decode down (80 tiles of 64x64, 216 iterations each) at 256 workgroups: 240 workgroups
    take one third of a tile each; C2's down (128 tiles, 64 iterations) keeps all 256."""
    plan = _lib.make_plan(64, 5120, 13824, 5120, _lib.BF16, "streamk", "erf", 256, -1, 8, m=16)
    assert (plan.down_tiles, plan.down_k_iters, plan.down_grid) == (80, 216, 240)
    plan = _lib.make_plan(4096, 1024, 4096, 1024, _lib.BF16, "streamk", "erf", 256, -1, 2)
    assert (plan.down_tiles, plan.down_k_iters, plan.down_grid) == (128, 64, 256)


def test_require_npu_is_the_reference_spelling_of_require_device():
    """Callers written against ops/host/inputs.py:56 pass require_npu; it means "the device
    the library runs on" and rejects CPU tensors the same way."""
    import torch
    from ffn_optim_amd.host.inputs import validate_tensors
    x, a, b = torch.zeros(2, 3).half(), torch.zeros(4, 3).half(), torch.zeros(3, 4).half()
    assert validate_tensors(x, a, b, require_npu=False).m == 2
    with pytest.raises(ValueError, match="requires ROCm GPU tensors"):
        validate_tensors(x, a, b, require_npu=True)


@pytest.mark.parametrize("damage", ["missing", "corrupt"])
def test_prepare_ffn_reports_an_unloadable_library(tmp_path, monkeypatch, damage):
    """A missing or corrupt libffn_mi355x.so surfaces from prepare_ffn as
    DependencyUnavailable (no fallback), before any device work (ops/host/dispatch.py:69-83)."""
    import torch
    from ffn_optim_amd import _lib, api
    from ffn_optim_amd.host import inputs
    from ffn_optim_amd.host.dispatch import DependencyUnavailable
    lib_path = tmp_path / "libffn_mi355x.so"
    if damage == "corrupt":
        lib_path.write_bytes(b"\x7fELF not really a shared object")
    monkeypatch.setattr(_lib, "LIBRARY_PATH", lib_path)
    monkeypatch.setattr(_lib, "_lib", None)
    # CPU tensors: let validation pass so that the library check is what fails
    monkeypatch.setattr(api, "validate_tensors",
                        lambda *a, **k: inputs.validate_tensors(*a, **dict(k, require_device=False)))
    x, a, b = torch.zeros(2, 16).half(), torch.zeros(64, 16).half(), torch.zeros(8, 64).half()
    with pytest.raises(DependencyUnavailable, match="libffn_mi355x.so"):
        api.prepare_ffn(x, a, b)


@pytest.mark.parametrize("plans", [False, True])
def test_prepare_ffn_reports_a_partial_library(tmp_path, monkeypatch, plans):
    """A library that loads but lacks entry points (a stale or partial build, here a gcc-built
    stand-in): without its planning entry points prepare_ffn reports DependencyUnavailable
    naming the missing symbol (ops/host/dispatch.py:69-83); with them but no launch entry
    point, binding the plan fails and prepare_ffn raises KernelCompilationError with the cause
    chained (ops/api.py:9-14, 82-88), before any input copy."""
    import subprocess
    import torch
    from ffn_optim_amd import _lib, api
    from ffn_optim_amd.host import inputs
    from ffn_optim_amd.host.dispatch import DependencyUnavailable
    lib_path = tmp_path / "libffn_mi355x.so"
    here = Path(__file__).resolve().parent
    cmd = ["gcc", "-shared", "-fPIC", "-Wall", "-Werror", "-I", str(here.parent / "include"),
           "-o", str(lib_path), str(here / "stubs" / "partial_abi.c")]
    if not plans:
        cmd.insert(1, "-DPARTIAL_ABI_NO_PLAN")
    subprocess.run(cmd, check=True)
    monkeypatch.setattr(_lib, "LIBRARY_PATH", lib_path)
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(api, "validate_tensors",
                        lambda *a, **k: inputs.validate_tensors(*a, **dict(k, require_device=False)))
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    copies = []
    monkeypatch.setattr(api, "prepare_storage", lambda *a, **k: copies.append(1))
    x, a, b = torch.zeros(2, 16).half(), torch.zeros(64, 16).half(), torch.zeros(8, 64).half()
    if not plans:
        with pytest.raises(DependencyUnavailable, match="ffn_mi355x_make_plan"):
            api.prepare_ffn(x, a, b)
    else:
        with pytest.raises(api.KernelCompilationError, match="ffn_mi355x_run") as info:
            api.prepare_ffn(x, a, b, down_impl="basic")
        assert isinstance(info.value.__cause__, RuntimeError)
    assert copies == []


def test_tile_keeps_the_reference_l1_names():
    from ffn_optim_amd.host.tiling import Tile
    t = Tile(256, 128, 64, 4, 3, 1)
    assert (t.l1_tm, t.l1_tn, t.l1_tk) == (256, 128, 64)


def test_compile_kernel_binds_a_plan_without_a_device():
    """compile_kernel (ops/host/dispatch.py:97-116) loads the library and binds the plan; its
    provenance names the entry point and the tile variants.  Binding touches no GPU."""
    from ffn_optim_amd.host.dispatch import compile_kernel
    from ffn_optim_amd.host.inputs import problem_from_shapes
    from ffn_optim_amd.host.tiling import make_plan
    for down in ("basic", "streamk"):
        plan = make_plan(problem_from_shapes((4096, 1024), (4096, 1024), (1024, 4096), "bfloat16"),
                         Selection("basic", down), 256)
        artifact, prov = compile_kernel(plan)
        assert callable(artifact)
        assert prov["down_impl"] == down and prov["entry_point"].startswith("ffn_mi355x_run")
        assert (prov["up_variant"], prov["down_variant"]) == (plan.up.variant, plan.down.variant)
        assert prov["version"].startswith("ffn_mi355x gfx950")


# The tile each measured workload runs on, as the design notes' tile table states it:
# (case id, down path) -> (up variant, down variant).
TUNED_ASSIGNMENTS = {
    ("c5_dit_bf16", "basic"): (22, 23), ("c5_dit_bf16", "streamk"): (22, 22),
    ("c2_aligned_bf16", "basic"): (22, 24), ("c2_aligned_bf16", "streamk"): (22, 23),
    ("c3_unaligned_fp16", "basic"): (18, 19), ("c3_unaligned_fp16", "streamk"): (18, 5),
    ("c4_decode_bf16", "basic"): (8, 20), ("c4_decode_bf16", "streamk"): (8, 19),
    ("c1_smoke_fp16", "basic"): (4, 20), ("c1_smoke_fp16", "streamk"): (4, 20),
    ("c5_tp8_shard_bf16", "basic"): (25, 25), ("c5_tp8_shard_bf16", "streamk"): (25, 22),
    ("c4_tp8_shard_bf16", "basic"): (15, 20), ("c4_tp8_shard_bf16", "streamk"): (19, 19),
}


@pytest.mark.parametrize("case_id,down", sorted(TUNED_ASSIGNMENTS))
def test_tuned_table_assignments(case_id, down):
    """Every workload plans to the variants the committed tuning table (and the design notes'
    tile table) assign it, at 256 workgroups."""
    from ffn_optim_amd.cases import get_case
    plan = make_plan(case_problem(get_case(case_id)), Selection("basic", down), 256)
    assert (plan.up.variant, plan.down.variant) == TUNED_ASSIGNMENTS[(case_id, down)]


def test_cost_model_takes_16x16_tiles_and_the_256x192_tile_where_measured():
    """Without the tuning table the cost model reaches the measured choices on the DiT-size FFN
    and its H/8 shard: the 256x256 tile of 16x16 blocks (22) over its 32x32 twin (12) for the
    full FFN's up (six tiles per CU), the 256x192 tile (25) for the shard's up, whose 192 tiles
    of 256x256 would leave 64 of 256 CUs idle."""
    from ffn_optim_amd.cases import get_case
    full = make_plan(case_problem(get_case("c5_dit_bf16")), Selection("basic", "streamk"), 256, tuned=False)
    shard = make_plan(case_problem(get_case("c5_tp8_shard_bf16")), Selection("basic", "basic"), 256, tuned=False)
    assert (full.up.variant, full.down.variant) == (22, 22)
    assert shard.up.variant == 25 and (shard.up.bm, shard.up.bn) == (256, 192)


def _untuned(m, k, h, down):
    p = problem_from_shapes((m, k), (h, k), (k, h), "bfloat16")
    return make_plan(p, Selection("basic", down), 256, tuned=False)


@pytest.mark.parametrize("m, k, h, up, down", [
    (1024, 5120, 13632, 22, 22),   # was 256x128: 160 tiles, 1.6 pieces a tile (now 28% faster)
    (3000, 1152, 4608, 22, 23),    # was 128x128: 216 tiles, 1.19 pieces a tile (now 36% faster)
    (1024, 3072, 12288, 25, 23),   # was 128x128: 192 tiles, 1.33 pieces a tile (now 20% faster)
])
def test_cost_model_keeps_stream_k_pieces_aligned(m, k, h, up, down):
    """A Stream-K down whose split tiles do not divide the grid has pieces starting at scattered
    depths of their tiles; the model streams those at the HBM rate, so the planner takes a tiling
    whose split tiles hold a whole number of pieces (every case measured faster than the plan
    chosen before, interleaved on the same inputs)."""
    plan = _untuned(m, k, h, "streamk")
    s = plan.schedule()
    assert (plan.up.variant, plan.down.variant) == (up, down)
    assert s["down_sk_tiles"] > 0 and s["down_grid"] % s["down_sk_tiles"] == 0, s


def test_forced_scattered_split_still_plans():
    """The scattered-pieces rule prices a tiling, it does not refuse it: a forced 256x128 down
    splits its 160 tiles over 256 workgroups as before.  The DiT-size FFN's automatic Stream-K
    down keeps split tiles that divide its grid (two pieces a tile)."""
    p = problem_from_shapes((1024, 5120), (13632, 5120), (5120, 13632), "bfloat16")
    forced = make_plan(p, Selection("basic", "streamk"), 256, up_variant=22, down_variant=23)
    s = forced.schedule()
    assert s["down_sk_tiles"] == 160 and s["down_grid"] == 256
    from ffn_optim_amd.cases import get_case
    full = make_plan(case_problem(get_case("c5_dit_bf16")), Selection("basic", "streamk"), 256, tuned=False)
    fs = full.schedule()
    assert fs["down_grid"] % fs["down_sk_tiles"] == 0


def test_256x128_tile_rated_lower_as_the_up_than_as_the_down():
    """The 256x128 tile is priced at 0.88 of the 256x256 tile per FLOP as the up GEMM and 0.95 as
    the down: DiT-XL's up (16384 x 1152 -> 4608) goes to the 256x192 tile (measured 4% faster),
    while a down it serves well keeps it (4096 x 5120 -> 13632 Basic, where the K-sliced 128x128
    tile measured 5.5% slower)."""
    assert _untuned(16384, 1152, 4608, "basic").up.variant == 25
    assert _untuned(4096, 5120, 13632, "basic").down.variant == 23
    assert _untuned(8192, 1024, 2752, "basic").up.variant == 25


@pytest.mark.parametrize("m, k, h, up_v, split", [
    (128, 4096, 16384, 5, False),   # 256 whole 64x128 tiles fill the grid: no split (measured -9%)
    (256, 2048, 8192, 5, False),    # the same at 256 rows (measured -17%)
    (64, 2048, 8192, 19, True),     # only 32x32 tiles fill it: the split 64x64 tile stays ahead
    (16, 5120, 1728, 20, True),     # decode shard: every tiling leaves half the grid idle
])
def test_split_up_only_where_no_tiling_fills_the_grid(m, k, h, up_v, split):
    """The automatic up GEMM is split along K only when no tiling of 64x64 or more would give more
    than half of the workgroups a whole tile; a forced variant still splits by its own tile count."""
    plan = _untuned(m, k, h, "basic")
    assert plan.up.variant == up_v and (plan.native.up_sk_tiles > 0) == split


@pytest.mark.parametrize("m, k, h, down, up_v, down_v", [
    (2048, 2048, 8192, "basic", 22, 24),   # load-bound K-sliced downs tie: v24 over v18 and v10
    (1000, 1024, 4096, "basic", 24, 19),   # the same tie on the up (measured -8%)
    (16, 3072, 12288, "basic", 19, 20),    # decode up on the K-sliced 64x64 tile (measured -13%)
    (512, 1024, 4096, "basic", 5, 19),     # its down on the K-sliced 64x64 tile, not 32x32 (-16%)
])
def test_cost_model_ties_go_to_the_faster_tile(m, k, h, down, up_v, down_v):
    """Where the load term bounds several tiles alike, a tile with refill-only waves is credited
    on its load rate too, and a tie goes to the tile of higher MFMA efficiency rather than the
    lower variant number; the K-sliced 32x32 decode tile is rated below the 64x64 one per FLOP."""
    plan = _untuned(m, k, h, down)
    assert (plan.up.variant, plan.down.variant) == (up_v, down_v)


def test_split_counter_stride_matches_header():
    """The Python mirror of the arrival-counter layout (used by the GPU tests that check which
    counter words a plan leaves zero) is the header's FFN_MI355X_SPLIT_COUNTER_WORDS, a 128-byte
    line of 32-bit counters that holds every tile wave of the widest tile."""
    header = (Path(__file__).resolve().parent.parent / "include" / "ffn_mi355x.h").read_text()
    words = int(re.search(r"#define FFN_MI355X_SPLIT_COUNTER_WORDS (\d+)", header).group(1))
    assert words == _lib.SPLIT_COUNTER_WORDS == 32
    info = _lib.variants()
    assert max(v["waves"] - v["refill_waves"] for v in info) <= words
