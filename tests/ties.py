"""Activations whose int8 quantization depends on rounding the product
x * (127 / amax) to f32 before the half-way offset is added.

For each such x the f32 product r lands exactly on a tie k + 0.5 (or on the
other side of it) while the exact product x * inv lies just across it: a
quantizer that fuses the multiply into the rounding addition (one FMA, as
HIP's default fp-contract allows) rounds them the other way. The CPU, and so
the reference, rounds the product first."""
import numpy as np

C = np.float32(float.fromhex("0x1.fffffep-2"))  # 0.5 - 2^-25, the device's offset


def fused_differs(v, inv):
    """Elementwise: does trunc(fl(fl(v*inv) + C)) differ from the fused
    trunc(fl(v*inv + C))? (v*inv + C is exact in f64: both terms fit.)"""
    v = np.asarray(v, np.float32)
    r = (v * inv).astype(np.float32)
    sep = np.trunc((r + np.copysign(C, r)).astype(np.float32))
    fused = np.trunc((v.astype(np.float64) * np.float64(inv) + np.copysign(np.float64(C), r)).astype(np.float32))
    return sep != fused


def near_ties(amax, count):
    """Up to count floats in (-amax, amax) whose quantization at this amax
    depends on the product's rounding (both signs)."""
    inv = np.float32(127.0) / np.float32(amax)
    k = np.arange(0, 127, dtype=np.float64) + 0.5
    v0 = (k / np.float64(inv)).astype(np.float32)
    cand = [v0]
    up, down = v0, v0
    for _ in range(48):
        up = np.nextafter(up, np.float32(np.inf))
        down = np.nextafter(down, np.float32(-np.inf))
        cand += [up, down]
    c = np.concatenate(cand)
    c = c[(c > 0) & (c < np.float32(amax))]
    hit = c[fused_differs(c, inv)]
    hit = np.concatenate([hit, -hit])
    return hit[:count]


def near_tie_x(n_groups, group, seed):
    """n_groups groups of `group` floats: element 0 the group's amax (a
    different one per group), the rest near-tie values for that amax (random
    normal values where too few exist)."""
    rng = np.random.default_rng(seed)
    out = np.empty((n_groups, group), np.float32)
    for g in range(n_groups):
        amax = np.float32(2.0 ** rng.uniform(-8, 8))
        vals = near_ties(amax, group - 1)
        fill = (rng.standard_normal(group - 1 - vals.size) * amax / 4).astype(np.float32)
        row = np.concatenate([[amax], vals, np.clip(fill, -amax, amax)]).astype(np.float32)
        out[g] = row
    return out.reshape(-1)
