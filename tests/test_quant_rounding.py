"""The GPU quantizers round r = x*127/amax with trunc(clamp(r + copysign(0.5 -
2^-25, r), -127, 127)) (q8_round in mdma_amd/csrc/kernels.h) where the oracle
(oracle/oracle.c orc_quantize_act, the reference's Q8_1 rule of
src/backend/rocm/kernels/kernels.hip:1102-1133) uses roundf and then clamps.
This checks that the two agree in IEEE float32 arithmetic over every value
near a half-integer in [-128, 128], every float in [0.25, 0.5), and a dense
sweep of bit patterns; and that adding 0.5 itself would not (at 0.5 - 2^-25)."""
import numpy as np


HALF_DOWN = np.float32(0.5) - np.float32(2.0 ** -25)


def device_rule(r, half=HALF_DOWN):
    t = (r + np.copysign(np.float32(half), r)).astype(np.float32)
    t = np.minimum(np.maximum(t, np.float32(-127)), np.float32(127))
    return np.trunc(t).astype(np.int32)


def oracle_rule(r):
    # roundf: half away from zero (np.round is half-to-even, so build it).
    a = np.floor(np.abs(r).astype(np.float64) + 0.5)
    q = np.copysign(a, r)
    return np.clip(q, -127, 127).astype(np.int32)


def test_rounding_identity_near_half_integers():
    k = np.arange(-128, 128, dtype=np.float32) + np.float32(0.5)
    vals = [k]
    for steps in range(1, 6):
        vals.append(np.nextafter(k, np.float32(np.inf)))
        vals.append(np.nextafter(k, np.float32(-np.inf)))
        k = vals[-1]
    r = np.concatenate(vals).astype(np.float32)
    r = np.concatenate([r, -r, np.float32([0.0, -0.0, 127.0, -127.0, 127.00002, -127.00002])])
    assert np.array_equal(device_rule(r), oracle_rule(r))


def test_rounding_identity_sweep():
    # Every 97th bit pattern of the positive floats below 128, and negatives.
    bits = np.arange(0, 0x43000000, 97, dtype=np.uint32)
    r = bits.view(np.float32)
    r = np.concatenate([r, -r])
    assert np.array_equal(device_rule(r), oracle_rule(r))


def test_rounding_identity_quarter_to_half():
    bits = np.arange(0x3E800000, 0x3F000000, dtype=np.uint32)  # every float in [0.25, 0.5)
    r = bits.view(np.float32)
    r = np.concatenate([r, -r])
    assert np.array_equal(device_rule(r), oracle_rule(r))


def test_adding_half_fails_below_one_half():
    # The plain r + 0.5 form rounds 0.5 - 2^-25 up to 1: the case the constant avoids.
    r = np.float32([0.5 - 2.0 ** -25])
    assert device_rule(r, np.float32(0.5))[0] == 1 and oracle_rule(r)[0] == 0 and device_rule(r)[0] == 0


def test_near_tie_activations_depend_on_the_product_rounding():
    """The fixture behind the GPU quantizer tests: near-tie activations exist
    in quantity, their oracle quantization is the product-first rounding,
    and a quantizer fusing the multiply into the offset addition (planted
    here on the CPU) disagrees with the oracle on them."""
    from oracle import ffi
    from ties import C, near_tie_x

    x = near_tie_x(16, 32, 5)
    q, d, _ = ffi.quantize_act(x, 32)
    xs = x.reshape(16, 32)
    amax = np.abs(xs).max(axis=1)
    inv = (np.float32(127.0) / amax).astype(np.float32)
    r = (xs * inv[:, None]).astype(np.float32)
    assert np.array_equal(q.reshape(16, 32), device_rule(r))
    fused = np.trunc((xs.astype(np.float64) * inv[:, None].astype(np.float64)
                      + np.copysign(np.float64(C), r)).astype(np.float32))
    fused = np.clip(fused, -127, 127).astype(np.int32)
    assert np.count_nonzero(fused != q.reshape(16, 32)) >= 32  # about 5 per group
