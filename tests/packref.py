"""Independent numpy restatement of the INT8 packer rule, used to pin the oracle.

Rule (QuantizedWeight::from_f32_transposed, src/ops/matmul.rs:1173-1202):
    max_abs = max over the row of |w|, NaN ignored, starting from 0
    scale   = max_abs / 127 (f32 division) if max_abs > 1e-8 else 1.0
    inv     = 1 / scale (f32 division)
    q       = round_half_away_from_zero(f32(w * inv)), clamped to [-127, 127], NaN -> 0
This implementation is vectorised numpy and rounds in float64 with floor(|x| + 0.5),
which is exact for every f32 input, so it shares no code path with the C oracle.
"""
import numpy as np


def pack_numpy(w_t):
    w = np.ascontiguousarray(w_t, dtype=np.float32)
    absw = np.abs(w)
    with np.errstate(invalid="ignore"):
        max_abs = np.where(np.isnan(absw), np.float32(0), absw).max(axis=1, initial=np.float32(0)).astype(np.float32)
    scale = np.where(max_abs > np.float32(1e-8), max_abs / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        inv = (np.float32(1.0) / scale).astype(np.float32)
        x = (w * inv[:, None]).astype(np.float32)
    xd = x.astype(np.float64)
    with np.errstate(invalid="ignore"):
        r = np.sign(xd) * np.floor(np.abs(xd) + 0.5)
        r = np.clip(r, -127.0, 127.0)
    q = np.where(np.isnan(r), 0.0, r).astype(np.int8)
    return q, scale
