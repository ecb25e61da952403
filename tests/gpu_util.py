"""Helpers shared by the GPU parity tests (seeded inputs, dtype handling)."""
import numpy as np
import torch

TORCH_DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
# Max-abs tolerance of attention outputs against the float64 closed form.
ATTN_TOL = {"bf16": 2e-2, "f16": 1e-2, "f32": 1e-4}


def to_dev(a, dtype, dev):
    return torch.as_tensor(np.asarray(a, dtype=np.float32)).to(dtype).to(dev)


def as_np(t):
    return t.detach().float().cpu().numpy()


def fill_store(store, rows_k, rows_v, dev):
    """Write natural-layout [len_r, 128] arrays into rows 0..n-1 of a store."""
    n = len(rows_k)
    Lmax = max([k.shape[0] for k in rows_k] + [1])
    src_k = torch.zeros((1, n, Lmax, 128), dtype=store.dtype, device=dev)
    src_v = torch.zeros_like(src_k)
    for r in range(n):
        L = rows_k[r].shape[0]
        if L:
            src_k[0, r, :L] = rows_k[r].to(store.dtype)
            src_v[0, r, :L] = rows_v[r].to(store.dtype)
    lens = [k.shape[0] for k in rows_k]
    store.write_rows(src_k, src_v, [(0, r) for r in range(n)], list(range(n)), lens)
    return src_k, src_v
