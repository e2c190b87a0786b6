"""Golden fixtures for the fused MoE path: seeded input recipes, the loader,
and (run as a script) the generator that writes the ``*.npz`` files here.

The reference commits no golden vectors (all of its tests are differential
against ``unfused_moe``, tests/conftest.py:58-137), so these fixtures are
written by this repository's CPU oracle from seeded inputs:

``c1_fp32.npz``   BASELINE configs[0]: N=256, D=128, ffn_dim=512, E=4, k=2,
                  softmax, swiglu, seed 0, x ~ N(0,1), weights ~ N(0,0.02);
                  the unfused fp32 forward (routing indices, weights, output).
``c1_bf16.npz``   the same inputs in bf16 through the fused oracle forward +
                  backward (upstream grad ~ N(0,1), seed 1), with the aux and
                  z losses; the weight gradients are kept as a seeded sample.
``routing.npz``   tie-heavy small-integer bf16 logits (N=300, E=16) and
                  Zipf-skewed logits (N=2048, E=64): top-k indices and weights
                  for k in (1, 2, 4, 8) under both gatings, per-expert counts,
                  the stable expert-sorted order and the capacity keep-mask.

Inputs are regenerated from their recipe (torch's CPU generator is
deterministic across machines); each fixture stores the SHA-256 of the
regenerated input bytes, so a changed recipe is caught.  bf16 arrays are
stored as their uint16 bit patterns.  Loading uses ``np.load`` with its default
``allow_pickle=False``.

Regenerate with ``python tests/golden/golden.py`` from the repository root.
"""

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

C1 = dict(N=256, D=128, ffn_dim=512, E=4, top_k=2)
TIE = dict(N=300, E=16)
SKEW = dict(N=2048, E=64)
KS = (1, 2, 4, 8)
CAPACITY_FACTOR = 1.0


def sha256(*tensors):
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.detach().contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


def c1_inputs():
    """x ~ N(0,1); gate, w_up, w_down ~ N(0, 0.02); seed 0 (fp32)."""
    g = torch.Generator().manual_seed(0)
    N, D, F, E = C1["N"], C1["D"], C1["ffn_dim"], C1["E"]
    x = torch.randn(N, D, generator=g)
    gate = torch.randn(E, D, generator=g) * 0.02
    w_up = torch.randn(E, F, D, generator=g) * 0.02
    w_down = torch.randn(E, D, F // 2, generator=g) * 0.02
    return x, gate, w_up, w_down


def c1_grad_out():
    g = torch.Generator().manual_seed(1)
    return torch.randn(C1["N"], C1["D"], generator=g)


def tie_logits():
    """Small integers in [-3, 3] as bf16: many exact ties per row."""
    g = torch.Generator().manual_seed(7)
    return torch.randint(-3, 4, (TIE["N"], TIE["E"]), generator=g).to(torch.bfloat16)


def skew_logits():
    """N(0,1) logits plus a per-expert bias 2*log(Zipf rank, s=1.1), as bf16:
    heavily skewed per-expert counts (the fine-grained, imbalanced config)."""
    g = torch.Generator().manual_seed(5)
    N, E = SKEW["N"], SKEW["E"]
    perm = torch.randperm(E, generator=g)
    bias = -2.0 * 1.1 * torch.log((perm + 1).float())
    return (torch.randn(N, E, generator=g) + bias).to(torch.bfloat16)


def weight_sample(shape, count=2048, seed=3):
    """Seeded flat indices of a weight-gradient sample."""
    g = torch.Generator().manual_seed(seed)
    n = int(np.prod(shape))
    return torch.randperm(n, generator=g)[:count].sort().values


def bits(t):
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def load(name):
    with np.load(os.path.join(HERE, name + ".npz")) as f:
        return {k: f[k] for k in f.files}


def _make_c1_fp32():
    from oracle.unfused import unfused_moe
    x, gate, wu, wd = c1_inputs()
    out, idx, w, _ = unfused_moe(x, gate, wu, wd, C1["top_k"])
    return dict(sha=np.array(sha256(x, gate, wu, wd)), topk_idx=idx.numpy().astype(np.int8),
                topk_w=w.float().numpy(), out=out.numpy())


def _make_c1_bf16():
    from oracle import fused as F_
    x, gate, wu, wd = (t.to(torch.bfloat16) for t in c1_inputs())
    go = c1_grad_out().to(torch.bfloat16)
    out, st = F_.forward(x, gate, wu, wd, C1["top_k"])
    gr = F_.backward(st, go)
    ls = F_.losses(st["logits"], st["topk_w"], st["topk_idx"], C1["E"], aux_loss_coeff=0.01,
                   z_loss_coeff=1e-3)
    su, sd = weight_sample(wu.shape, seed=3), weight_sample(wd.shape, seed=4)
    return dict(sha=np.array(sha256(x, gate, wu, wd, go)),
                topk_idx=st["topk_idx"].numpy().astype(np.int8), topk_w=st["topk_w"].numpy(),
                logits=bits(st["logits"]), out=bits(out), d_hidden=bits(gr["hidden"]),
                d_gate=bits(gr["gate"]), w_up_sample=su.numpy(),
                d_w_up_sample=bits(gr["w_up"].reshape(-1)[su]), w_down_sample=sd.numpy(),
                d_w_down_sample=bits(gr["w_down"].reshape(-1)[sd]),
                aux_loss=np.float32(ls["aux_loss"].item()), z_loss=np.float32(ls["z_loss"].item()))


def _make_routing():
    from oracle import routing as R
    res = {}
    for tag, logits in (("tie", tie_logits()), ("skew", skew_logits())):
        N, E = logits.shape
        res[f"{tag}_logits"] = bits(logits)
        res[f"{tag}_sha"] = np.array(sha256(logits))
        lf = logits.float().numpy()
        for k in KS:
            for gating in ("softmax", "sigmoid"):
                w, idx = R.route(lf, k, gating)
                res[f"{tag}_{gating}_k{k}_idx"] = idx.astype(np.int8)
                res[f"{tag}_{gating}_k{k}_w"] = w.astype(np.float32)
            idx = res[f"{tag}_softmax_k{k}_idx"].astype(np.int64)
            order, counts, starts, rank = R.stable_permutation(idx, E)
            res[f"{tag}_k{k}_counts"] = counts.astype(np.int32)
            res[f"{tag}_k{k}_order"] = order.astype(np.int16)
            cap = R.expert_capacity(N, E, k, CAPACITY_FACTOR)
            res[f"{tag}_k{k}_capacity"] = np.int32(cap)
            res[f"{tag}_k{k}_keep"] = R.capacity_keep(idx, E, cap)
            res[f"{tag}_k{k}_max_tokens"] = np.int32(R.estimate_max_tokens(N, k, E))
    return res


MAKERS = {"c1_fp32": _make_c1_fp32, "c1_bf16": _make_c1_bf16, "routing": _make_routing}


def main():
    root = os.path.dirname(os.path.dirname(HERE))
    if root not in sys.path:
        sys.path.insert(0, root)
    torch.set_num_threads(1)
    for name, make in MAKERS.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **make())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
