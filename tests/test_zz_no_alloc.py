"""The allocation-free gate-gradient entry point (ffmoe_gate_grad_noalloc)
against the workspace one (ffmoe_gate_grad), called through the C ABI:
bit-identical results on two calls in a row, the second with a smaller
input (the shared scratch keeps the first call's partials, which the second
must not read), and a host-side rejection of sizes beyond the scratch."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(N, D, E, seed):
    g = torch.Generator().manual_seed(seed)
    gl = (torch.randn(N, E, generator=g) * 0.1).to(torch.bfloat16).cuda()
    x = torch.randn(N, D, generator=g).to(torch.bfloat16).cuda()
    return gl, x


def _with_workspace(L, gl, x, N, D, E):
    ws = torch.empty(int(L.load().ffmoe_gate_grad_workspace_bytes(N, D, E)), dtype=torch.uint8,
                     device="cuda")
    out = torch.empty(E, D, dtype=torch.bfloat16, device="cuda")
    L.call("ffmoe_gate_grad", L.ptr(gl), L.ptr(x), N, D, E, L.ptr(ws), L.ptr(out), L.stream_ptr())
    return out


def _no_alloc(L, gl, x, N, D, E):
    out = torch.empty(E, D, dtype=torch.bfloat16, device="cuda")
    L.call("ffmoe_gate_grad_noalloc", L.ptr(gl), L.ptr(x), N, D, E, L.ptr(out), L.stream_ptr())
    return out


def test_gate_grad_noalloc_matches_workspace_variant_twice():
    from flashfusedmoe_amd import _lib as L
    for (N, D, E, seed) in ((8192, 1024, 8, 1), (1000, 264, 12, 2)):
        gl, x = _inputs(N, D, E, seed)
        ref = _with_workspace(L, gl, x, N, D, E)
        got = _no_alloc(L, gl, x, N, D, E)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (N, D, E)
        exp = (gl.float().t() @ x.float())
        assert ((got.float() - exp).norm() / exp.norm()).item() < 1e-2


def test_gate_grad_noalloc_rejects_sizes_beyond_its_scratch():
    from flashfusedmoe_amd import _lib as L
    cap = int(L.load().ffmoe_gate_grad_noalloc_max_bytes())
    N, D, E = 1 << 20, 4096, 32  # 8192 chunks x 32 x 4096 x 4 bytes = 4 GiB of partials
    assert int(L.load().ffmoe_gate_grad_workspace_bytes(N, D, E)) > cap
    with pytest.raises(L.FFMoEError, match="at most"):
        # rejected on the host before any launch: the pointers are never read
        L.call("ffmoe_gate_grad_noalloc", 0, 0, N, D, E, 0, L.stream_ptr())
