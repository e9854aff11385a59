"""numpy <-> device tensor helpers for the GPU parity tests."""
import numpy as np
import torch


def to_dev(a: np.ndarray, dev) -> torch.Tensor:
    """uint16 arrays are bf16 bit patterns and become bfloat16 tensors."""
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def say(msg: str) -> None:
    """Names the case before a GPU step, flushed, so a fault still shows it."""
    print(f"[gpu-case] {msg}", flush=True)


def device_case(dev, seed, B, hq, hkv, d, ctx, bs=16, dtype=torch.bfloat16):
    """Large seeded case generated on the device (torch Philox), so the
    config-sized tests do not spend minutes in host RNG.  Returns device
    tensors and host copies: (q, k, v, tables, ctx) on device, the pools as
    numpy (uint16 bf16 bits or float32)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    need = [(int(L) + bs - 1) // bs for L in ctx]
    nb = int(sum(need))
    k = torch.randn((nb, hkv, bs, d), generator=g, device=dev).to(dtype)
    v = torch.randn((nb, hkv, bs, d), generator=g, device=dev).to(dtype)
    q = torch.randn((B, hq, d), generator=g, device=dev)
    perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32).cpu().numpy()
    tables = np.full((B, max(need)), -1, np.int32)
    o = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[o:o + n]
        o += n
    ctx = np.asarray(ctx, np.int32)
    return (q, k, v, to_dev(tables, dev), to_dev(ctx, dev)), (to_np(q), to_np(k), to_np(v),
                                                              tables, ctx)
