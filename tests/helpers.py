"""Shared helpers for the GPU parity tests."""
import numpy as np
import torch


def rel_l2(got, ref) -> float:
    if isinstance(got, torch.Tensor):
        got = got.detach().float().cpu().numpy()
    got = np.asarray(got, dtype=np.float64).reshape(np.shape(ref))
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


def to_dev(a, dtype, shape=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if shape is not None:
        t = t.reshape(shape)
    return t.to("cuda:0").to(dtype).contiguous()


def announce(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
