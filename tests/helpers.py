"""Shared helpers for the decode-attention tests."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def to_np(t: torch.Tensor) -> np.ndarray:
    """CPU numpy copy; bfloat16 becomes its exact float32 value, fp16 stays fp16."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.float().numpy()          # every bf16 value is exactly representable
    return t.numpy()


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def load_golden(name: str):
    """(arrays dict, dtype str) of a fixture; q/kv_data as float16, or float32 for bf16."""
    z = dict(np.load(GOLDEN / f"{name}.npz", allow_pickle=False))
    dtype = str(z["dtype"])
    if dtype == "bf16":
        z["q_f32"] = bf16_bits_to_f32(z["q"])
        z["kv_f32"] = bf16_bits_to_f32(z["kv_data"])
    else:
        z["q_f32"] = z["q"].astype(np.float32)
        z["kv_f32"] = z["kv_data"].astype(np.float32)
    return z, dtype


def golden_to_torch(z, dtype: str, device: str):
    """Fixture inputs as device tensors in the fixture's dtype."""
    if dtype == "bf16":
        q = torch.from_numpy(z["q"].view(np.int16).copy()).view(torch.bfloat16)
        kv = torch.from_numpy(z["kv_data"].view(np.int16).copy()).view(torch.bfloat16)
    else:
        q = torch.from_numpy(z["q"].copy())
        kv = torch.from_numpy(z["kv_data"].copy())
    tabs = [torch.from_numpy(z[k].astype(np.int32)) for k in
            ("kv_indptr", "kv_indices", "kv_last_page_len")]
    return (q.to(device), kv.to(device), *[t.to(device) for t in tabs])


def err_stats(out: torch.Tensor, ref: np.ndarray):
    """(max_abs, mean_abs) of out (any dtype, any device) vs a numpy reference."""
    o = out.detach().float().cpu().numpy().astype(np.float64)
    d = np.abs(o - np.asarray(ref, np.float64))
    return float(d.max()) if d.size else 0.0, float(d.mean()) if d.size else 0.0


def check_partials(po, pm, pl, O, m, l, dtype):
    """Pass-1 partials vs the exact ones. m is the split max of the scaled scores and l
    the fp32 sum of exp(s - m). P.V weights p enter the MFMA as hi + lo parts of the
    element type (relative error 2^-22 for fp16, 2^-17 for bf16), so O is compared
    through the normalised O / l, with |V| <= ~5 in these inputs."""
    pm, pl, po = pm.cpu().numpy(), pl.cpu().numpy(), po.cpu().numpy()
    np.testing.assert_allclose(pm, m, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(pl, l, rtol=1e-5, atol=1e-6)
    live = l > 0
    np.testing.assert_allclose(po[live] / pl[live][:, None], O[live] / l[live][:, None],
                               rtol=0, atol=1e-4 if dtype == torch.float16 else 2e-4)
    assert (po[~live] == 0).all()
