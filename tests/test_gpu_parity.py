"""GPU parity: the HIP path (libffmoe.so) against the CPU oracle on identical
seeded inputs.  Integer/index results (top-k indices, counts, the token
permutation) must be bit-exact; floating-point results must match within the
bf16 tolerance of gpu_helpers.check_close (rtol 2e-2, atol 2e-3, fp32
accumulation)."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import check_close, cuda, expected_rows, probe_lds_transpose, seeded
from oracle import fused as F_
from oracle import routing as R

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _lib():
    from flashfusedmoe_amd import _lib as L
    L.load()
    yield L
    L.set_lds_transpose(True)


# --- the gfx950 LDS transpose read the MN-contiguous GEMM operands rely on -----

def test_lds_transpose_read_lane_layout():
    got = probe_lds_transpose()
    for lane in range(64):
        g, i = lane // 16, lane % 16
        col = (g & 1) * 16 + i
        rows = [(g >> 1) * 8 + q for q in range(4)]
        assert list(got[lane]) == [r * 64 + col for r in rows], f"lane {lane}: {list(got[lane])}"


# --- routing -------------------------------------------------------------------

def _tie_heavy_logits(N, E, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-3, 4, (N, E), generator=g).to(torch.bfloat16)


@pytest.mark.parametrize("E,k", [(8, 2), (4, 1), (16, 4), (7, 3), (64, 8), (256, 8), (256, 16), (33, 5)])
@pytest.mark.parametrize("gating", ["softmax", "sigmoid"])
@pytest.mark.parametrize("ties", [False, True])
def test_topk_routing_bit_exact(E, k, gating, ties):
    from flashfusedmoe_amd.kernels import fused_topk_routing
    N = 1000
    if ties:
        logits = _tie_heavy_logits(N, E, E * 7 + k)
    else:
        g = torch.Generator().manual_seed(E + k)
        logits = torch.randn(N, E, generator=g).to(torch.bfloat16)
    w, idx = fused_topk_routing(logits.cuda(), gating, k)
    rw, ridx = R.route(logits.float().numpy(), k, gating)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("N,D,E", [(8192, 1024, 8), (777, 256, 64), (4096, 7168, 256), (5, 64, 16)])
def test_gate_logits_and_routing(N, D, E):
    """The fused MFMA gate GEMM rounds an fp32 sum to bf16.  Each logit is
    within one bf16 ulp of the exact product plus the fp32 summation error
    bound (2^-20 * sum|x_i g_i| covers D <= 16K terms), most are the
    correctly rounded value, and routing of the produced logits is
    bit-exact."""
    from flashfusedmoe_amd import ops
    x, gate, _, _ = seeded(N, D, 16, E, seed=N + E)
    k = min(8, E)
    outs = ops.route(x.cuda(), gate.cuda(), None, k, 0, R.estimate_max_tokens(N, k, E), 0.0, 0.0,
                     False)
    logits, idx, w = outs[0].cpu(), outs[1].cpu(), outs[2].cpu()
    exact64 = x.double() @ gate.double().t()
    absum = x.double().abs() @ gate.double().abs().t()
    ulp = torch.exp2(torch.floor(torch.log2(exact64.abs().clamp_min(1e-30))) - 7)
    err = (logits.double() - exact64).abs()
    assert bool((err <= ulp + 2.0 ** -20 * absum).all()), "gate logits outside the rounding bound"
    rounded = exact64.to(torch.bfloat16)
    assert (logits != rounded).double().mean().item() < 0.02
    rw, ridx = R.route(logits.float().numpy(), k, "softmax")
    assert np.array_equal(idx.numpy(), ridx)
    np.testing.assert_allclose(w.numpy(), rw, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("N,E,k,mt,cap", [(8192, 8, 2, None, False), (1000, 64, 8, 40, False),
                                           (1000, 64, 8, 40, True), (3, 8, 2, None, False),
                                           (4096, 256, 8, None, False), (777, 7, 3, None, False),
                                           (2000, 33, 5, 100, True), (16384, 64, 8, None, False)])
def test_permutation_bit_exact(N, E, k, mt, cap):
    from flashfusedmoe_amd import ops
    D = 128
    x, gate, wu, wd = seeded(N, D, 64, E, seed=N * 3 + E)
    if mt is None:
        mt = R.estimate_max_tokens(N, k, E)
    xg, gg, wug, wdg = cuda(x, gate, wu, wd)
    (logits, idx, tw, lse, counts, offsets, tile_off, stats, istats, ws, _aux, _z) = ops.route(
        xg, gg, None, k, 0, mt, 0.0, 0.0, False)
    out, tw2, row_of, xs, up, act, down, _, _ = ops.experts_forward(
        xg, wug, wdg, idx, tw, counts, offsets, tile_off, ws, k, 0, mt, cap, True)
    exp_rows, exp_counts, exp_off = expected_rows(idx.cpu().numpy(), E, mt, cap)
    assert np.array_equal(counts.cpu().numpy(), exp_counts)
    assert np.array_equal(offsets.cpu().numpy(), exp_off)
    assert np.array_equal(row_of.cpu().numpy(), exp_rows)
    own = exp_rows >= 0
    j = np.nonzero(own)[0]
    assert torch.equal(xs.cpu()[exp_rows[own]], x[j // k])
    from flashfusedmoe_amd import _lib as L
    bm = L.gemm_tile_rows(N * k, E)
    tiles = -(-np.minimum(exp_counts, mt) // bm)
    assert np.array_equal(tile_off.cpu().numpy()[1:], np.cumsum(tiles))


# --- expert GEMMs against a plain fp32 PyTorch reference ------------------------

def _groups(E, sizes, D, H, seed):
    g = torch.Generator().manual_seed(seed)
    rows = int(sum(sizes))
    xs = torch.randn(rows, D, generator=g).to(torch.bfloat16)
    wu = (torch.randn(E, 2 * H, D, generator=g) * D ** -0.5).to(torch.bfloat16)
    wd = (torch.randn(E, D, H, generator=g) * H ** -0.5).to(torch.bfloat16)
    off = np.zeros(E + 1, dtype=np.int32)
    off[1:] = np.cumsum(sizes)
    return xs, wu, wd, off


# the skewed C2-sized case has more tiles than CUs, so the persistent
# schedule splits tiles along K between blocks ("sk"); "dp" is one block per
# tile, "elementwise" the element-wise LDS read variant of that
@pytest.mark.parametrize("sizes,D,H", [
    ([300, 0, 128, 1, 513, 64, 0, 127], 256, 192),
    ([2048] * 8, 1024, 2048),
    ([2100, 1900, 2300, 1700, 2048, 2048, 2500, 1800], 1024, 2048),
    ([2100, 1900, 2300, 1700, 2048, 2048, 2500, 1800], 4096, 512),
    ([5, 17, 0, 260], 96, 40),
    # 256-row tiles with H not a multiple of the 64-column dgrad+GLU tiles
    ([700, 0, 900], 256, 200),
])
@pytest.mark.parametrize("mode", ["sk", "dp", "elementwise"])
def test_grouped_gemms_against_fp32(sizes, D, H, mode, _lib):
    L = _lib
    E = len(sizes)
    xs, wu, wd, off = _groups(E, sizes, D, H, seed=sum(sizes) + D)
    T = xs.shape[0]
    bm = L.gemm_tile_rows(T, E)
    tiles = np.zeros(E + 1, dtype=np.int32)
    tiles[1:] = np.cumsum([-(-s // bm) for s in sizes])
    dev = "cuda"
    xs_g, wu_g, wd_g = cuda(xs, wu, wd)
    off_g = torch.from_numpy(off).to(dev)
    til_g = torch.from_numpy(tiles).to(dev)
    st = L.stream_ptr()
    L.set_lds_transpose(mode != "elementwise")
    wsb = L.gemm_workspace(torch.device(dev), st)
    ws = wsb.data_ptr() if mode == "sk" else None
    up = torch.empty(T, 2 * H, dtype=torch.bfloat16, device=dev)
    act = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    down = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    L.call("ffmoe_gemm_up_glu", xs_g.data_ptr(), wu_g.data_ptr(), off_g.data_ptr(), til_g.data_ptr(),
           bm, E, T, D, H, 0, up.data_ptr(), act.data_ptr(), ws, st)
    L.call("ffmoe_gemm_down", act.data_ptr(), wd_g.data_ptr(), off_g.data_ptr(), til_g.data_ptr(),
           bm, E, T, H, D, down.data_ptr(), ws, st)
    g = torch.Generator().manual_seed(5)
    wgo = torch.randn(T, D, generator=g).to(torch.bfloat16).cuda()
    gup = torch.empty(T, 2 * H, dtype=torch.bfloat16, device=dev)
    L.call("ffmoe_gemm_dgrad_glu", wgo.data_ptr(), wd_g.data_ptr(), up.data_ptr(), off_g.data_ptr(),
           til_g.data_ptr(), bm, E, T, D, H, 0, gup.data_ptr(), ws, st)
    ghb = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    L.call("ffmoe_gemm_dgrad", gup.data_ptr(), wu_g.data_ptr(), off_g.data_ptr(), til_g.data_ptr(),
           bm, E, T, H, D, ghb.data_ptr(), ws, st)
    dwd = torch.empty(E, D, H, dtype=torch.bfloat16, device=dev)
    L.call("ffmoe_gemm_wgrad", wgo.data_ptr(), act.data_ptr(), off_g.data_ptr(), E, D, H,
           dwd.data_ptr(), st)
    dwu = torch.empty(E, 2 * H, D, dtype=torch.bfloat16, device=dev)
    L.call("ffmoe_gemm_wgrad", gup.data_ptr(), xs_g.data_ptr(), off_g.data_ptr(), E, 2 * H, D,
           dwu.data_ptr(), st)
    torch.cuda.synchronize()
    L.set_lds_transpose(True)
    # every flag consumed (the workspace is reusable) and no wait timed out
    assert int(wsb[:8192].view(torch.int32).abs().sum().item()) == 0

    # fp32 reference per expert on the GPU, from the kernels' own bf16 inputs
    f = lambda t: t.float()  # noqa: E731
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            ref_up = f(xs_g[a:b]) @ f(wu_g[e]).t()
            check_close(up[a:b], ref_up, f"up[e={e}]")
            gg, uu = f(up[a:b, :H]), f(up[a:b, H:])
            check_close(act[a:b], torch.nn.functional.silu(gg) * uu, f"act[e={e}]")
            check_close(down[a:b], f(act[a:b]) @ f(wd_g[e]).t(), f"down[e={e}]")
            gact = (f(wgo[a:b]) @ f(wd_g[e])).to(torch.bfloat16).float()
            s = torch.sigmoid(gg)
            ref_gu = gact * gg * s
            ref_gg = gact * uu * (s * (1 + gg * (1 - s)))
            check_close(gup[a:b], torch.cat([ref_gg, ref_gu], 1), f"gup[e={e}]")
            check_close(ghb[a:b], f(gup[a:b]) @ f(wu_g[e]), f"ghb[e={e}]")
            check_close(dwd[e], f(wgo[a:b]).t() @ f(act[a:b]), f"dW_down[e={e}]")
            check_close(dwu[e], f(gup[a:b]).t() @ f(xs_g[a:b]), f"dW_up[e={e}]")
        else:
            assert dwd[e].abs().max().item() == 0 and dwu[e].abs().max().item() == 0


@pytest.mark.parametrize("sizes,D,H", [
    ([2100, 1900, 2300, 1700, 2048, 2048, 2500, 1800], 1024, 2048),
    # many small experts (128-row tiles) and K >= 4096 for both GEMMs: long
    # stream-K tails where a block publishes partials for two cut tiles
    ([100 + (37 * e) % 61 for e in range(32)], 4096, 2048),
])
def test_persistent_schedule_is_deterministic(sizes, D, H, _lib):
    # a cut tile's two partials are summed the same way whichever block
    # finishes second: three runs agree bit for bit, and the workspace flags
    # are left zero
    L = _lib
    E = len(sizes)
    xs, wu, wd, off = _groups(E, sizes, D, H, seed=77)
    T = xs.shape[0]
    bm = L.gemm_tile_rows(T, E)
    tiles = np.zeros(E + 1, dtype=np.int32)
    tiles[1:] = np.cumsum([-(-s // bm) for s in sizes])
    xs_g, wu_g, wd_g = cuda(xs, wu, wd)
    off_g = torch.from_numpy(off).cuda()
    til_g = torch.from_numpy(tiles).cuda()
    st = L.stream_ptr()
    wsb = L.gemm_workspace(torch.device("cuda"), st)
    outs = []
    for _ in range(3):
        up = torch.empty(T, 2 * H, dtype=torch.bfloat16, device="cuda")
        act = torch.empty(T, H, dtype=torch.bfloat16, device="cuda")
        ghb = torch.empty(T, D, dtype=torch.bfloat16, device="cuda")
        L.call("ffmoe_gemm_up_glu", xs_g.data_ptr(), wu_g.data_ptr(), off_g.data_ptr(),
               til_g.data_ptr(), bm, E, T, D, H, 0, up.data_ptr(), act.data_ptr(), wsb.data_ptr(), st)
        L.call("ffmoe_gemm_dgrad", up.data_ptr(), wu_g.data_ptr(), off_g.data_ptr(),
               til_g.data_ptr(), bm, E, T, H, D, ghb.data_ptr(), wsb.data_ptr(), st)
        torch.cuda.synchronize()
        outs.append((up.cpu(), act.cpu(), ghb.cpu()))
    for run in outs[1:]:
        for a, b in zip(outs[0], run):
            assert torch.equal(a, b)
    assert int(wsb[:8192].view(torch.int32).abs().sum().item()) == 0


# The fused up+down launch against the two separate launches (down with no
# workspace: one block per tile, as in the fused schedule, so the outputs are
# the same bits), with and without a dense group after the routed rows.
# Cases with 128-row tiles take the two-launch path inside the entry point.
@pytest.mark.parametrize("sizes,D,H,shared_rows,act", [
    ([2100, 1900, 2300, 1700, 2048, 2048, 2500, 1800], 1024, 2048, 0, 0),
    ([2048] * 8, 1024, 2048, 8192, 0),
    ([0, 1500, 0, 600], 256, 320, 0, 0),
    ([700, 900], 256, 64, 513, 0),
    ([300, 0, 128, 1, 513, 64, 0, 127], 256, 192, 0, 0),
    # the other activations through the same epilogues (whole and half tiles)
    ([1900, 2200, 2048, 1700], 512, 1024, 1000, 1),
    ([1900, 2200, 2048, 1700], 512, 1024, 0, 2),
    ([300, 0, 128, 1, 513, 64, 0, 127], 256, 192, 0, 3),
])
def test_fused_up_down_matches_two_launches(sizes, D, H, shared_rows, act, _lib):
    L = _lib
    E = len(sizes)
    xs, wu, wd, off = _groups(E, sizes, D, H, seed=31 + sum(sizes))
    T = xs.shape[0]
    bm = L.gemm_tile_rows(T, E)
    print(f"fused up+down: sizes={sizes} D={D} H={H} shared={shared_rows} act={act} tile_rows={bm}", flush=True)
    tiles = np.zeros(E + 1, dtype=np.int32)
    tiles[1:] = np.cumsum([-(-s // bm) for s in sizes])
    xs_g, wu_g, wd_g = cuda(xs, wu, wd)
    off_g = torch.from_numpy(off).cuda()
    til_g = torch.from_numpy(tiles).cuda()
    st = L.stream_ptr()
    wsb = L.gemm_workspace(torch.device("cuda"), st)
    g = torch.Generator().manual_seed(9)
    N = shared_rows
    sx = torch.randn(N, D, generator=g).to(torch.bfloat16).cuda()
    sgu = (torch.randn(2 * H, D, generator=g) * D ** -0.5).to(torch.bfloat16).cuda()
    sdn = (torch.randn(D, H, generator=g) * H ** -0.5).to(torch.bfloat16).cuda()

    def outputs():
        bf = dict(dtype=torch.bfloat16, device="cuda")
        o = [torch.empty(T, 2 * H, **bf), torch.empty(T, H, **bf), torch.empty(T, D, **bf),
             torch.empty(N, 2 * H, **bf), torch.empty(N, H, **bf), torch.empty(N, D, **bf)]
        gu = L.dense_group(sx, sgu, o[4], N, act, c2=o[3]) if N else None
        gd = L.dense_group(o[4], sdn, o[5], N, 0) if N else None
        return o, (ctypes.byref(gu) if gu else None), (ctypes.byref(gd) if gd else None)

    ref, gu, gd = outputs()
    L.call("ffmoe_gemm_up_glu_shared", xs_g.data_ptr(), wu_g.data_ptr(), off_g.data_ptr(), til_g.data_ptr(),
           bm, E, T, D, H, act, ref[0].data_ptr(), ref[1].data_ptr(), gu, None, st)
    L.call("ffmoe_gemm_down_shared", ref[1].data_ptr(), wd_g.data_ptr(), off_g.data_ptr(), til_g.data_ptr(),
           bm, E, T, H, D, ref[2].data_ptr(), gd, None, st)
    for _ in range(3):
        got, gu, gd = outputs()
        L.call("ffmoe_gemm_up_down_shared", xs_g.data_ptr(), wu_g.data_ptr(), wd_g.data_ptr(), off_g.data_ptr(),
               til_g.data_ptr(), bm, E, T, D, H, act, got[0].data_ptr(), got[1].data_ptr(), got[2].data_ptr(),
               gu, gd, wsb.data_ptr(), st)
        torch.cuda.synchronize()
        for name, a, b in zip(["up", "act", "down", "shared up", "shared act", "shared down"], got, ref):
            assert torch.equal(a, b), name
    # the schedule's words are left zero and no wait timed out
    assert int(wsb[:8192].view(torch.int32).abs().sum().item()) == 0
    assert int(wsb[-65536:].view(torch.int32).abs().sum().item()) == 0
    # and the result is the product: the routed rows against fp32
    f = lambda t: t.float()  # noqa: E731
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            check_close(ref[2][a:b], f(ref[1][a:b]) @ f(wd_g[e]).t(), f"down[e={e}]")
    if N:
        check_close(ref[5], f(ref[4]) @ f(sdn).t(), "shared down")


# The fused dgrad + up-side wgrad launch against the two separate launches
# bit for bit (dgrad with no workspace: whole tiles, as in the fused
# schedule; the wgrad with the workspace, which cuts a large dense group's K
# in two either way), with and without a dense group; the last case takes
# the two-launch path inside the entry point (2H not a multiple of 64).
@pytest.mark.parametrize("sizes,D,H,shared_rows", [
    ([2100, 1900, 2300, 1700, 2048, 2048, 2500, 1800], 1024, 2048, 0),
    ([2048] * 8, 1024, 2048, 8192),
    ([100 + (37 * e) % 61 for e in range(32)], 512, 256, 0),
    ([0, 1500, 0, 600], 256, 320, 700),
    ([700, 900], 256, 104, 0),
    # few rows per expert (the eight-wave launch) with a dense group cut in K
    ([100 + (37 * e) % 61 for e in range(16)], 512, 256, 5000),
])
def test_fused_dgrad_wgrad_matches_two_launches(sizes, D, H, shared_rows, _lib):
    L = _lib
    E = len(sizes)
    H2 = 2 * H
    g = torch.Generator().manual_seed(41 + sum(sizes))
    T = sum(sizes)
    bm = L.gemm_tile_rows(T, E)
    print(f"fused dgrad+wgrad: sizes={sizes[:4]}... E={E} D={D} H={H} shared={shared_rows} tile_rows={bm}",
          flush=True)
    off = np.zeros(E + 1, dtype=np.int32)
    off[1:] = np.cumsum(sizes)
    tiles = np.zeros(E + 1, dtype=np.int32)
    tiles[1:] = np.cumsum([-(-s // bm) for s in sizes])
    gup = torch.randn(T, H2, generator=g).to(torch.bfloat16).cuda()
    xs = torch.randn(T, D, generator=g).to(torch.bfloat16).cuda()
    wu = (torch.randn(E, H2, D, generator=g) * D ** -0.5).to(torch.bfloat16).cuda()
    off_g = torch.from_numpy(off).cuda()
    til_g = torch.from_numpy(tiles).cuda()
    st = L.stream_ptr()
    wsb = L.gemm_workspace(torch.device("cuda"), st)
    N = shared_rows
    sgup = torch.randn(N, H2, generator=g).to(torch.bfloat16).cuda()
    sx = torch.randn(N, D, generator=g).to(torch.bfloat16).cuda()
    sgu = (torch.randn(H2, D, generator=g) * D ** -0.5).to(torch.bfloat16).cuda()

    def outputs():
        bf = dict(dtype=torch.bfloat16, device="cuda")
        o = [torch.empty(T, D, **bf), torch.empty(E, H2, D, **bf), torch.empty(N, D, **bf),
             torch.empty(H2 if N else 0, D, **bf)]
        gd = L.dense_group(sgup, sgu, o[2], N, 0) if N else None
        gw = L.dense_group(sgup, sx, o[3], N, 0) if N else None
        return o, (ctypes.byref(gd) if gd else None), (ctypes.byref(gw) if gw else None)

    ref, gd, gw = outputs()
    L.call("ffmoe_gemm_wgrad_shared", gup.data_ptr(), xs.data_ptr(), off_g.data_ptr(), E, H2, D,
           ref[1].data_ptr(), gw, wsb.data_ptr(), st)
    L.call("ffmoe_gemm_dgrad_shared", gup.data_ptr(), wu.data_ptr(), off_g.data_ptr(), til_g.data_ptr(), bm,
           E, T, H, D, ref[0].data_ptr(), gd, None, st)
    first = None
    for _ in range(3):
        got, gd, gw = outputs()
        L.call("ffmoe_gemm_dgrad_wgrad_shared", gup.data_ptr(), wu.data_ptr(), xs.data_ptr(), off_g.data_ptr(),
               til_g.data_ptr(), bm, E, T, H, D, got[0].data_ptr(), got[1].data_ptr(), gd, gw, wsb.data_ptr(),
               st)
        torch.cuda.synchronize()
        for name, a, b in zip(["ghb", "dw_up", "shared ghb", "shared dw_up"], got, ref):
            assert torch.equal(a, b), name
        first = got
    assert int(wsb[:8192].view(torch.int32).abs().sum().item()) == 0
    assert int(wsb[-65536:].view(torch.int32).abs().sum().item()) == 0
    f = lambda t: t.float()  # noqa: E731
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            check_close(ref[0][a:b], f(gup[a:b]) @ f(wu[e]), f"ghb[e={e}]")
            check_close(ref[1][e], f(gup[a:b]).t() @ f(xs[a:b]), f"dW_up[e={e}]")
        else:
            assert ref[1][e].abs().max().item() == 0
    if N:
        check_close(first[2], f(sgup) @ f(sgu), "shared ghb")
        check_close(ref[3], f(sgup).t() @ f(sx), "shared dW_up")


@pytest.mark.parametrize("k", [2, 4, 8, 16])
@pytest.mark.parametrize("E", [3, 8, 32])
def test_dx_reduce_and_gate_grad_against_fp32(E, k, _lib):
    # dx[n] = bf16(bf16(sum_s ghb[row]) + bf16(gl[n] . gate)); dgate = gl^T x
    L = _lib
    N, D = 1000, 264
    g = torch.Generator().manual_seed(E)
    T = N * k
    ghb = torch.randn(T, D, generator=g).to(torch.bfloat16)
    gl = (torch.randn(N, E, generator=g) * 0.1).to(torch.bfloat16)
    gate = (torch.randn(E, D, generator=g) * 0.05).to(torch.bfloat16)
    x = torch.randn(N, D, generator=g).to(torch.bfloat16)
    row_of = torch.randperm(T, generator=g).to(torch.int32)
    row_of[::37] = L.ROW_DROPPED
    row_of[5::53] = L.ROW_ALIAS0
    ghb_g, gl_g, gate_g, x_g, ro_g = cuda(ghb, gl, gate, x, row_of)
    st = L.stream_ptr()
    dx = torch.empty(N, D, dtype=torch.bfloat16, device="cuda")
    L.call("ffmoe_dx_reduce", ghb_g.data_ptr(), ro_g.data_ptr(), gl_g.data_ptr(), gate_g.data_ptr(),
           N, D, E, k, dx.data_ptr(), st)
    part = torch.empty(int(L.load().ffmoe_gate_grad_workspace_bytes(N, D, E)), dtype=torch.uint8,
                       device="cuda")
    dgate = torch.empty(E, D, dtype=torch.bfloat16, device="cuda")
    L.call("ffmoe_gate_grad", gl_g.data_ptr(), x_g.data_ptr(), N, D, E, part.data_ptr(),
           dgate.data_ptr(), st)
    torch.cuda.synchronize()
    src = row_of.long().clone()
    src[row_of == L.ROW_ALIAS0] = 0
    valid = (row_of != L.ROW_DROPPED).view(N, k, 1).double()
    rows = ghb.double()[src.clamp(min=0)].view(N, k, D) * valid
    s = rows.sum(1).to(torch.bfloat16).double()
    a = (gl.double() @ gate.double()).to(torch.bfloat16).double()
    check_close(dx.cpu(), (s + a), "dx")
    check_close(dgate.cpu(), gl.double().t() @ x.double(), "dgate")


@pytest.mark.parametrize("E", [3, 8, 32])
def test_dx_reduce_dropped_slots_add_nothing(E, _lib):
    # The same problem as k = 2 and as k = 16 with slots 2..15 dropped is
    # the same arithmetic in the same order (dropped slots add nothing), so
    # the results must be the same bits.
    L = _lib
    N, D = 777, 136
    g = torch.Generator().manual_seed(100 + E)
    ghb = torch.randn(2 * N, D, generator=g).to(torch.bfloat16).cuda()
    gl = (torch.randn(N, E, generator=g) * 0.1).to(torch.bfloat16).cuda()
    gate = (torch.randn(E, D, generator=g) * 0.05).to(torch.bfloat16).cuda()
    ro2 = torch.randperm(2 * N, generator=g).to(torch.int32)
    ro2[::29] = L.ROW_DROPPED
    ro16 = torch.full((N, 16), L.ROW_DROPPED, dtype=torch.int32)
    ro16[:, :2] = ro2.view(N, 2)
    st = L.stream_ptr()
    outs = []
    for k, ro in ((2, ro2.cuda()), (16, ro16.reshape(-1).cuda())):
        dx = torch.empty(N, D, dtype=torch.bfloat16, device="cuda")
        L.call("ffmoe_dx_reduce", ghb.data_ptr(), ro.data_ptr(), gl.data_ptr(), gate.data_ptr(), N, D, E, k,
               dx.data_ptr(), st)
        torch.cuda.synchronize()
        outs.append(dx)
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("N,D,E", [(1000, 256, 48), (4096, 1024, 64), (700, 7168, 256), (333, 64, 40)])
def test_mfma_gate_products_against_fp64(N, D, E):
    """Above 32 experts gl @ gate (ffmoe_gate_dx) and gl^T x
    (ffmoe_gate_grad's MFMA split-K path) run on the MFMA GEMM pipeline with
    fp32 accumulation and one bf16 rounding: within one bf16 ulp of the
    exact product plus the fp32 summation bound, and at most 2% of them not
    the correctly rounded value.  E = 40 and 48 exercise the zero padding."""
    from flashfusedmoe_amd import ops
    g = torch.Generator().manual_seed(N + E)
    gl = (torch.randn(N, E, generator=g) * 0.1).to(torch.bfloat16)
    gate = (torch.randn(E, D, generator=g) * 0.05).to(torch.bfloat16)
    x = torch.randn(N, D, generator=g).to(torch.bfloat16)
    dx = ops.gate_dx(gl.cuda(), gate.cuda()).cpu()
    dgate = ops.gate_grad(gl.cuda(), x.cuda()).cpu()
    for name, got, a, b in (("gl @ gate", dx, gl.double(), gate.double()),
                            ("gl^T x", dgate, gl.double().t(), x.double())):
        exact = a @ b
        absum = a.abs() @ b.abs()
        ulp = torch.exp2(torch.floor(torch.log2(exact.abs().clamp_min(1e-30))) - 7)
        err = (got.double() - exact).abs()
        assert bool((err <= ulp + 2.0 ** -20 * absum).all()), f"{name} outside the rounding bound"
        assert (got != exact.to(torch.bfloat16)).double().mean().item() < 0.02, name


@pytest.mark.parametrize("N,D,E", [(16384, 2048, 64), (4096, 7168, 256), (1000, 512, 100)])
def test_mfma_gate_logits_split_k(N, D, E):
    """The MFMA gate GEMM (split along D, fp32 partials added in a fixed
    order): within the rounding bound of the exact product, almost always the
    correctly rounded bf16, bitwise repeatable.  Also reports how many
    logits are not the correctly rounded value and how many tokens' top-k
    differ from routing the exact logits (ties of nearly equal logits)."""
    from flashfusedmoe_amd import ops
    x, gate, _, _ = seeded(N, D, 16, E, seed=N + D + E)
    lg = ops.gate_logits(x.cuda(), gate.cuda())
    lg2 = ops.gate_logits(x.cuda(), gate.cuda())
    assert torch.equal(lg, lg2)
    lg = lg.cpu()
    exact64 = x.double() @ gate.double().t()
    absum = x.double().abs() @ gate.double().abs().t()
    ulp = torch.exp2(torch.floor(torch.log2(exact64.abs().clamp_min(1e-30))) - 7)
    err = (lg.double() - exact64).abs()
    assert bool((err <= ulp + 2.0 ** -20 * absum).all()), "logits outside the rounding bound"
    not_rounded = (lg != exact64.to(torch.bfloat16)).double().mean().item()
    assert not_rounded < 0.02
    k = 8
    _, idx_gpu = R.route(lg.float().numpy(), k)
    # what an exact GEMM hands the router: the correctly rounded bf16 logits
    _, idx_rn = R.route(exact64.to(torch.bfloat16).float().numpy(), k)
    _, idx_exact = R.route(exact64.float().numpy(), k)
    differ = int((idx_gpu != idx_rn).any(axis=1).sum())
    differ_exact = int((idx_gpu != idx_exact).any(axis=1).sum())
    print(f"\n[parity report] N={N} D={D} E={E}: {not_rounded:.4%} of logits not the correctly "
          f"rounded bf16; {differ} of {N} tokens route differently from the correctly rounded "
          f"logits' top-{k} ({differ_exact} from the unrounded fp64 logits' top-{k}, where bf16 "
          f"ties are broken by value)")
    assert differ <= 0.002 * N


def test_many_experts_gate_products_use_mfma_path():
    # E above the fused-kernel limit: gl @ gate and gl^T x run on the MFMA
    # pipeline (ffmoe_gate_dx, ffmoe_gate_grad's split-K path)
    N, D, ffn, E, k = 512, 128, 256, 64, 4
    x, gate, wu, wd = seeded(N, D, ffn, E, seed=64)
    go = torch.randn(N, D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    out, losses, grads = _run_layer(x, gate, wu, wd, k, go, allow_dropped_tokens=True)
    from flashfusedmoe_amd import ops
    logits = ops.route(x.cuda(), gate.cuda(), None, k, 0, 1, 0.0, 0.0, False)[0].cpu()
    ref, st = F_.forward(x, gate, wu, wd, k, allow_dropped_tokens=True, logits=logits)
    check_close(out, ref, "output")
    gr = F_.backward(st, go)
    check_close(grads[0], gr["hidden"], "grad hidden")
    check_close(grads[1], gr["gate"], "grad gate", atol=2e-3 * max(1.0, gr["gate"].abs().max().item()))


def test_transpose_and_elementwise_lds_reads_agree(_lib):
    """Both LDS read paths of the MN-contiguous operands give identical bits."""
    L = _lib
    sizes = [333, 0, 700, 64]
    E, D, H = 4, 512, 256
    xs, wu, wd, off = _groups(E, sizes, D, H, seed=9)
    T = xs.shape[0]
    g = torch.Generator().manual_seed(1)
    gup = torch.randn(T, 2 * H, generator=g).to(torch.bfloat16).cuda()
    off_g = torch.from_numpy(off).cuda()
    res = []
    for tr in (True, False):
        L.set_lds_transpose(tr)
        c = torch.empty(E, 2 * H, D, dtype=torch.bfloat16, device="cuda")
        L.call("ffmoe_gemm_wgrad", gup.data_ptr(), xs.cuda().data_ptr(), off_g.data_ptr(), E, 2 * H,
               D, c.data_ptr(), L.stream_ptr())
        res.append(c)
    L.set_lds_transpose(True)
    assert torch.equal(res[0], res[1])


@pytest.mark.parametrize("E,seed", [(80, 0), (300, 1)])
def test_wgrad_skewed_counts_against_fp32(E, seed, _lib):
    """One expert far above the mean row count (plus ties and empty experts)
    sends the wgrad launch down its heaviest-first, XCD-sliced tile order.
    Every expert still matches an fp32 product, empty experts are zero, and
    the heavy expert's tiles are bit-identical to a launch of that expert
    alone (the order changes which block runs a tile, not its arithmetic)."""
    L = _lib
    rng = np.random.default_rng(seed)
    sizes = rng.integers(0, 48, E)
    sizes[:6] = 17
    sizes[6:10] = 0
    heavy = int(rng.integers(10, E))
    sizes[heavy] = 3000
    assert 2 * sizes.max() * E >= 3 * sizes.sum()
    M, Nc = 264, 520  # partial edge tiles on both sides
    T = int(sizes.sum())
    off = np.zeros(E + 1, dtype=np.int32)
    off[1:] = np.cumsum(sizes)
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(T, M, generator=g).to(torch.bfloat16).cuda()
    b = torch.randn(T, Nc, generator=g).to(torch.bfloat16).cuda()
    off_g = torch.from_numpy(off).cuda()
    c = torch.full((E, M, Nc), float("nan"), dtype=torch.bfloat16, device="cuda")
    L.call("ffmoe_gemm_wgrad", a.data_ptr(), b.data_ptr(), off_g.data_ptr(), E, M, Nc, c.data_ptr(),
           L.stream_ptr())
    ref = torch.zeros(E, M, Nc, device="cuda")
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi > lo:
            ref[e] = a[lo:hi].float().t() @ b[lo:hi].float()
    torch.cuda.synchronize()
    check_close(c, ref, "dW (skewed counts)")
    assert c[torch.from_numpy(sizes == 0).cuda()].abs().max().item() == 0
    lo, hi = int(off[heavy]), int(off[heavy + 1])
    one_off = torch.tensor([0, hi - lo], dtype=torch.int32, device="cuda")
    c1 = torch.empty(1, M, Nc, dtype=torch.bfloat16, device="cuda")
    L.call("ffmoe_gemm_wgrad", a[lo:hi].contiguous().data_ptr(), b[lo:hi].contiguous().data_ptr(),
           one_off.data_ptr(), 1, M, Nc, c1.data_ptr(), L.stream_ptr())
    torch.cuda.synchronize()
    assert torch.equal(c[heavy], c1[0])


# --- the whole layer against the oracle -----------------------------------------

def _run_layer(x, gate, wu, wd, k, go, **kw):
    from flashfusedmoe_amd import fused_moe
    leaves = [t.cuda().requires_grad_(True) for t in (x, gate, wu, wd)]
    out, losses = fused_moe(*leaves, top_k=k, **kw)
    loss = (out.float() * go.cuda().float()).sum()
    for key in ("aux_loss", "z_loss"):
        if key in losses and losses[key].requires_grad:
            loss = loss + losses[key]
    loss.backward()
    return out.detach().cpu(), losses, [t.grad.cpu() for t in leaves]


@pytest.mark.parametrize("activation", ["swiglu", "geglu", "relu_squared"])
@pytest.mark.parametrize("gating", ["softmax", "sigmoid"])
@pytest.mark.parametrize("N,D,ffn,E,k", [(256, 128, 512, 4, 2), (1000, 256, 384, 16, 4)])
def test_layer_forward_backward_matches_oracle(activation, gating, N, D, ffn, E, k):
    x, gate, wu, wd = seeded(N, D, ffn, E, seed=N + E + k)
    go = torch.randn(N, D, generator=torch.Generator().manual_seed(99)).to(torch.bfloat16)
    aux_c, z_c = 0.01, 0.001
    out, losses, grads = _run_layer(x, gate, wu, wd, k, go, activation=activation, gating=gating,
                                    aux_loss_coeff=aux_c, z_loss_coeff=z_c,
                                    allow_dropped_tokens=True)
    # routing is pinned to the GPU's bf16 logits (identical-logits contract)
    from flashfusedmoe_amd import ops
    logits = ops.route(x.cuda(), gate.cuda(), None, k, 0, 1, 0.0, 0.0, False)[0].cpu()
    ref, st = F_.forward(x, gate, wu, wd, k, activation=activation, gating=gating,
                         allow_dropped_tokens=True, logits=logits)
    check_close(out, ref, "output")
    ls = F_.losses(logits, st["topk_w"], st["topk_idx"], E, gating=gating, aux_loss_coeff=aux_c,
                   z_loss_coeff=z_c)
    torch.testing.assert_close(losses["aux_loss"].cpu(), ls["aux_loss"].float(), rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(losses["z_loss"].cpu(), ls["z_loss"].float(), rtol=1e-4, atol=1e-6)
    assert losses["aux_loss"].requires_grad == (gating == "sigmoid")

    gr = F_.backward(st, go)
    lg = F_.loss_grads(logits, st["topk_idx"], E, gating, aux_c, z_c).to(torch.bfloat16)
    exp_hidden = (gr["hidden"].float() + F_.gemm(lg, gate).float())
    exp_gate = (gr["gate"].float() + F_.gemm(lg.t().contiguous(), x).float())
    check_close(grads[0], exp_hidden, "grad hidden")
    check_close(grads[1], exp_gate, "grad gate", atol=2e-3 * max(1.0, exp_gate.abs().max().item()))
    check_close(grads[2], gr["w_up"], "grad w_up")
    check_close(grads[3], gr["w_down"], "grad w_down")


def test_metrics_match_oracle():
    from flashfusedmoe_amd import fused_moe
    N, D, ffn, E, k = 640, 128, 256, 8, 2
    x, gate, wu, wd = seeded(N, D, ffn, E, seed=3)
    out, losses = fused_moe(*cuda(x, gate, wu, wd), top_k=k, return_metrics=True,
                            allow_dropped_tokens=True, capacity_factor=0.5)
    from flashfusedmoe_amd import ops
    logits = ops.route(x.cuda(), gate.cuda(), None, k, 0, 1, 0.0, 0.0, False)[0].cpu()
    w, idx = F_.apply_routing(logits, "softmax", k)
    ls = F_.losses(logits, w, idx, E, return_metrics=True, capacity_factor=0.5, top_k=k)
    assert torch.equal(losses["tokens_per_expert"].cpu(), ls["tokens_per_expert"])
    assert losses["tokens_per_expert"].dtype == torch.int32
    assert losses["max_expert_load"].item() == ls["max_expert_load"].item()
    assert losses["min_expert_load"].item() == ls["min_expert_load"].item()
    assert abs(losses["expert_load_imbalance"].item() - ls["expert_load_imbalance"].item()) < 1e-5
    assert losses["dropped_token_count"].item() == ls["dropped_token_count"].item()
    assert abs(losses["dropped_token_fraction"].item() - ls["dropped_token_fraction"].item()) < 1e-6


def test_capacity_matches_oracle():
    N, D, ffn, E, k = 512, 128, 256, 4, 2
    x, gate, wu, wd = seeded(N, D, ffn, E, seed=21, gate_scale=0.2)
    go = torch.randn(N, D, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    out, _, grads = _run_layer(x, gate, wu, wd, k, go, capacity_factor=1.0)
    from flashfusedmoe_amd import ops
    logits = ops.route(x.cuda(), gate.cuda(), None, k, 0, 1, 0.0, 0.0, False)[0].cpu()
    ref, st = F_.forward(x, gate, wu, wd, k, capacity_factor=1.0, logits=logits)
    assert not bool(st["keep"].all())
    check_close(out, ref, "output")
    gr = F_.backward(st, go)
    check_close(grads[0], gr["hidden"], "grad hidden")
    check_close(grads[2], gr["w_up"], "grad w_up")
    check_close(grads[3], gr["w_down"], "grad w_down")


def test_overflow_raises_and_alias_semantics():
    from flashfusedmoe_amd import fused_moe
    N, D, ffn, E, k = 64, 64, 128, 4, 1
    x, gate, wu, wd = seeded(N, D, ffn, E, seed=42)
    gate = gate.clone()
    gate[0] += 1.0
    with pytest.raises(RuntimeError, match="MoE routing overflow"):
        fused_moe(*cuda(x, gate, wu, wd), top_k=k, max_tokens_per_expert=16)
    out, _ = fused_moe(*cuda(x, gate, wu, wd), top_k=k, max_tokens_per_expert=16,
                       allow_dropped_tokens=True)
    from flashfusedmoe_amd import ops
    logits = ops.route(x.cuda(), gate.cuda(), None, k, 0, 1, 0.0, 0.0, False)[0].cpu()
    ref, st = F_.forward(x, gate, wu, wd, k, max_tokens_per_expert=16, allow_dropped_tokens=True,
                         logits=logits)
    assert not bool(st["keep"].all())
    check_close(out.cpu(), ref, "output with overflow")


@pytest.mark.parametrize("N,E,k", [(1, 4, 2), (4, 16, 2), (32, 4, 1), (32, 8, 3), (32, 8, 4)])
def test_edge_cases_match_oracle(N, E, k):
    # tests/test_production.py:488-616 analogues
    D, ffn = 64, 128
    x, gate, wu, wd = seeded(N, D, ffn, E, seed=N + E + k)
    go = torch.randn(N, D, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    out, _, grads = _run_layer(x, gate, wu, wd, k, go, allow_dropped_tokens=True)
    from flashfusedmoe_amd import ops
    logits = ops.route(x.cuda(), gate.cuda(), None, k, 0, 1, 0.0, 0.0, False)[0].cpu()
    ref, st = F_.forward(x, gate, wu, wd, k, allow_dropped_tokens=True, logits=logits)
    check_close(out, ref, "output")
    gr = F_.backward(st, go)
    check_close(grads[0], gr["hidden"], "grad hidden")
    check_close(grads[2], gr["w_up"], "grad w_up")


def test_empty_experts():
    # tests/test_production.py:502-522: experts 4..7 receive nothing
    N, D, ffn, E, k = 16, 64, 128, 8, 2
    x, gate, wu, wd = seeded(N, D, ffn, E, seed=7)
    gate = gate.clone()
    gate[4:] = 0.0
    gate[:4] *= 100.0
    go = torch.randn(N, D, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    out, _, grads = _run_layer(x, gate, wu, wd, k, go, allow_dropped_tokens=True)
    from flashfusedmoe_amd import ops
    logits = ops.route(x.cuda(), gate.cuda(), None, k, 0, 1, 0.0, 0.0, False)[0].cpu()
    ref, st = F_.forward(x, gate, wu, wd, k, allow_dropped_tokens=True, logits=logits)
    check_close(out, ref, "output")
    gr = F_.backward(st, go)
    check_close(grads[2], gr["w_up"], "grad w_up")
    check_close(grads[3], gr["w_down"], "grad w_down")
    # experts that received no token get exactly zero weight gradients
    unused = torch.bincount(st["topk_idx"].view(-1), minlength=E) == 0
    if bool(unused.any()):
        assert grads[2][unused].abs().max().item() == 0.0


def test_recompute_is_bitwise_identical():
    # tests/test_production.py:258-311
    N, D, ffn, E, k = 512, 128, 256, 8, 2
    x, gate, wu, wd = seeded(N, D, ffn, E, seed=11)
    go = torch.randn(N, D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    a = _run_layer(x, gate, wu, wd, k, go, allow_dropped_tokens=True)
    b = _run_layer(x, gate, wu, wd, k, go, allow_dropped_tokens=True, recompute_activations=True)
    assert torch.equal(a[0], b[0])
    for ga, gb in zip(a[2], b[2]):
        assert torch.equal(ga, gb)


def test_run_twice_bitwise_deterministic():
    N, D, ffn, E, k = 2048, 256, 512, 16, 4
    x, gate, wu, wd = seeded(N, D, ffn, E, seed=12)
    go = torch.randn(N, D, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    a = _run_layer(x, gate, wu, wd, k, go, aux_loss_coeff=0.01, z_loss_coeff=0.001,
                   allow_dropped_tokens=True)
    b = _run_layer(x, gate, wu, wd, k, go, aux_loss_coeff=0.01, z_loss_coeff=0.001,
                   allow_dropped_tokens=True)
    assert torch.equal(a[0], b[0])
    for ga, gb in zip(a[2], b[2]):
        assert torch.equal(ga, gb)


def test_expert_bias_selection_only():
    """expert_bias shifts selection only; weights use unbiased logits
    (fused_moe.py:163-179)."""
    from flashfusedmoe_amd import fused_moe, ops
    N, D, ffn, E, k = 512, 128, 256, 16, 4
    x, gate, wu, wd = seeded(N, D, ffn, E, seed=13)
    bias = -2.2 * torch.log(torch.randperm(E, generator=torch.Generator().manual_seed(1)).float() + 1)
    outs = ops.route(x.cuda(), gate.cuda(), bias.cuda(), k, 0, N * k, 0.0, 0.0, False)
    logits, idx, w = outs[0].cpu(), outs[1].cpu(), outs[2].cpu()
    sel = logits.float() + bias
    ridx, _ = R.topk_select(sel.numpy(), k)
    assert np.array_equal(idx.numpy(), ridx)
    rw = torch.softmax(logits.float().gather(1, idx), -1)
    torch.testing.assert_close(w, rw, rtol=2e-6, atol=1e-7)
    out, _ = fused_moe(*cuda(x, gate, wu, wd), top_k=k, expert_bias=bias.cuda(),
                       allow_dropped_tokens=True)
    ref, _ = F_.forward(x, gate, wu, wd, k, allow_dropped_tokens=True, logits=logits,
                        expert_bias=bias)
    check_close(out.cpu(), ref, "output with expert_bias")
