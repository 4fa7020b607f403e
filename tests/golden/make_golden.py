"""Writes the golden fixtures tests/golden/{clip,lit}_*.npz.

Expected values come from the library route, independently of the oracle's
fixed-max formulas: F.normalize(dim=1) + dense logits + F.cross_entropy in
fp64, gradients by torch.autograd.  Inputs are stored as float32 values (bf16
cases hold bf16-representable values), so GPU tests feed exactly these values.

    python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))

# name, path, n, d, temperature, normalized_inputs, stable, bf16, correlated
CASES = [
    ("clip_n1_d8", "clip", 1, 8, 0.07, False, False, False, False),
    ("clip_n7_d5", "clip", 7, 5, 0.07, False, False, False, False),
    ("clip_n130_d33", "clip", 130, 33, 0.05, False, False, False, False),
    ("clip_n256_d64_normed", "clip", 256, 64, 0.07, True, False, False, True),
    ("clip_n200_d16_stable", "clip", 200, 16, 0.1, False, True, False, False),
    ("clip_n300_d48_bf16", "clip", 300, 48, 0.07, True, False, True, True),
    ("lit_n9_d6", "lit", 9, 6, 0.07, False, False, False, False),
    ("lit_n129_d40", "lit", 129, 40, 0.07, False, False, False, False),
    ("lit_n256_d64_stable_normed", "lit", 256, 64, 0.05, True, True, False, True),
]


def make_inputs(n, d, normalized, bf16, correlated, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(n, d, generator=g)
    if correlated:
        a = F.normalize(a, dim=1)
        b = F.normalize(a + 0.5 * torch.randn(n, d, generator=g), dim=1)
    else:
        b = torch.randn(n, d, generator=g)
        if normalized:
            a, b = F.normalize(a, dim=1), F.normalize(b, dim=1)
    if bf16:
        a, b = a.bfloat16().float(), b.bfloat16().float()
    return a.contiguous(), b.contiguous()


def library_route(path, a, b, t, normalized, stable):
    a64 = a.double().requires_grad_(True)
    b64 = b.double().requires_grad_(path == "clip")
    xh = a64 if normalized else F.normalize(a64, dim=1)
    yh = b64 if normalized else F.normalize(b64, dim=1)
    s = xh @ yh.T / t
    lab = torch.arange(a.shape[0])
    loss = F.cross_entropy(s, lab)
    if path == "clip":
        loss = 0.5 * (loss + F.cross_entropy(s.T, lab))
    loss.backward()
    scale = (a.shape[0] * t) ** 0.5 if stable else 1.0
    da = (a64.grad * scale).numpy()
    db = (b64.grad * scale).numpy() if path == "clip" else None
    return loss.item(), da, db


def main():
    for k, (name, path, n, d, t, normalized, stable, bf16, correlated) in enumerate(CASES):
        a, b = make_inputs(n, d, normalized, bf16, correlated, seed=1000 + k)
        loss, da, db = library_route(path, a, b, t, normalized, stable)
        out = dict(a=a.numpy(), b=b.numpy(), temperature=np.float64(t), normalized_inputs=np.bool_(normalized),
                   stable=np.bool_(stable), bf16=np.bool_(bf16), loss=np.float64(loss), da=da)
        if db is not None:
            out["db"] = db
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **out)
        print(f"{name}: loss={loss:.10f}")


if __name__ == "__main__":
    main()
