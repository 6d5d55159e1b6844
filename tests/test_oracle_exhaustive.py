"""Exhaustive checks that pin the C checker's fp16 arithmetic and prove the
cheaper quantiser arithmetic of the HIP append kernel (csrc/quant.h)
bit-identical to the reference quantiser (torch_eager_kv.py:75-86)."""
import numpy as np
import torch

from oracle import c_oracle


def test_f16_to_f32_all_65536_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = c_oracle.f16_bits_to_f32(torch.from_numpy(bits.view(np.int16))).numpy()
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.array_equal(np.isinf(got), np.isinf(want))


def test_f32_to_f16_round_nearest_even():
    # every fp16 value, every midpoint between neighbours (exact ties), the
    # floats adjacent to each midpoint, overflow edges and random floats
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h[:-1] + h[1:]) / 2
    m32 = mids.astype(np.float32)
    cands = np.concatenate([
        h.astype(np.float32), m32, np.nextafter(m32, np.float32(np.inf)),
        np.nextafter(m32, np.float32(0)), np.float32([65504, 65519.99, 65520, 65536, 1e30, 2.0 ** -25,
                                                      2.0 ** -24, 3 * 2.0 ** -26, 0.0]),
        np.random.default_rng(0).standard_normal(1 << 20).astype(np.float32) * 100,
    ])
    cands = np.concatenate([cands, -cands])
    want = cands.astype(np.float16).view(np.uint16)
    got = c_oracle.f32_to_f16_bits(torch.from_numpy(cands)).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_scale_multiply_by_one_seventh_is_exact():
    # RN16(max(RN32(a * RN32(1/7)), 2^-14)) == RN16(max(RN32(a / 7), 2^-14))
    # for all 31744 finite non-negative fp16 amax values.
    assert c_oracle.check_scale_mul() == 0


def test_quantiser_is_exact_for_every_reachable_input():
    # Every scale the quantiser can emit x every fp16 x with |x| up to the
    # largest group amax giving that scale, with the reciprocal correctly
    # rounded or off by up to two floats either way.
    for rvariant in (0, -1, 1, -2, 2):
        assert c_oracle.check_quant_grid(rvariant) == 0


def test_quantiser_check_detects_planted_mistakes():
    # Past the group amax the missing clamp shows; rounding in one step
    # instead of two gets exact half-way cases wrong.  The exhaustive check
    # must see both.
    assert c_oracle.check_quant_grid(0, mode=1) > 0
    assert c_oracle.check_quant_grid(0, mode=2) > 0


def test_shift_and_add_packing_is_exact():
    # All 15^8 code tuples of a 32-dim group pack to pack_int4's nibbles;
    # a bias off by one does not.
    assert c_oracle.check_pack_sum() == 0
    assert c_oracle.check_pack_sum(1) > 0
