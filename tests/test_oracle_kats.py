"""Pin the CPU checkers (oracle/) against the reference's own known-answer
tests and scenarios (tests/test_correctness.py and tests/test_attention.py of
Hunter2030ZeRo/Iris-Kernel) and against closed forms.

Every KAT runs on both restatements: the torch one (oracle.torch_eager_*)
and the plain-C one (oracle.c_oracle)."""
import json
from pathlib import Path

import pytest
import torch

from oracle import c_oracle
from oracle.torch_eager_attention import dequantize_int4_groupwise, unpack_int4
from oracle.torch_eager_kv import apply_rope, pack_int4, quantize_int4_groupwise, torch_eager_append

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def c_append(case):
    kw = {k: case[k] for k in ("rotary_dim", "group_size", "page_size")}
    c_oracle.append(case["key"], case["value"], case["positions"], case["slot_mapping"],
                    case["cos_cache"], case["sin_cache"], case["k_data"], case["v_data"],
                    case["k_scale"], case["v_scale"], **kw)


# ---------------------------------------------------------------- RoPE KATs
def test_rope_pos_zero_is_identity():
    # test_correctness.py:18-31
    x = torch.randn(2, 3, 8)
    out = apply_rope(x, torch.ones(2, 1, 4), torch.zeros(2, 1, 4), rotary_dim=8)
    torch.testing.assert_close(out, x)


def test_rope_quarter_turn():
    # test_correctness.py:34-49: [1,2,3,4] with cos=0, sin=1 -> [-3,-4,1,2]
    kat = GOLDEN["rope_quarter_turn"]
    x = torch.tensor([[kat["x"]]])
    out = apply_rope(x, torch.zeros(1, 1, 2), torch.ones(1, 1, 2), rotary_dim=4)
    torch.testing.assert_close(out, torch.tensor([[kat["expected"]]]))


def test_rope_passthrough_dims():
    # test_correctness.py:307-324
    x = torch.randn(2, 3, 8)
    out = apply_rope(x, torch.zeros(2, 1, 2), torch.ones(2, 1, 2), rotary_dim=4)
    torch.testing.assert_close(out[..., 4:], x[..., 4:])


def test_rope_rotation_closed_form():
    # fp32: rotate-half RoPE by angle a maps (x1, x2) to (x1 cos a - x2 sin a, x2 cos a + x1 sin a),
    # preserves each pair's norm, and is undone by angle -a.
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 2, 16, generator=g, dtype=torch.float64)
    ang = torch.rand(5, 1, 8, generator=g, dtype=torch.float64) * 6.28
    y = apply_rope(x, ang.cos(), ang.sin(), rotary_dim=16)
    back = apply_rope(y, ang.cos(), -ang.sin(), rotary_dim=16)
    torch.testing.assert_close(back, x)
    torch.testing.assert_close(x[..., :8] ** 2 + x[..., 8:] ** 2, y[..., :8] ** 2 + y[..., 8:] ** 2)


# ------------------------------------------------------------ quantise KATs
def test_quantize_known_values():
    # test_correctness.py:52-72: [-7,-3,0,7], group 4 -> same codes, scale 1.0
    kat = GOLDEN["quantize"]
    q, s = quantize_int4_groupwise(torch.tensor([[kat["x"]]]), group_size=4)
    assert q.dtype == torch.int8
    assert q.flatten().tolist() == kat["q"]
    assert s.flatten().tolist() == kat["scale"]


def test_quantize_zero_group_is_finite():
    # test_correctness.py:75-82; the scale is finfo(fp16).tiny = 2^-14
    q, s = quantize_int4_groupwise(torch.zeros(2, 3, 8, dtype=torch.float16), group_size=4)
    assert torch.all(q == 0)
    assert torch.all(s == 2.0 ** -14)


def test_quantize_closed_form_and_ties():
    # Scale 1.0 (amax 7): x = k + 1/2 rounds half to even.
    x = torch.tensor([[7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]], dtype=torch.float16)
    q, s = quantize_int4_groupwise(x, group_size=8)
    assert s.item() == 1.0
    assert q.flatten().tolist() == [7, 0, 2, 2, 0, -2, -2, 4]
    # scale = RN16(amax / 7); codes reconstruct within half a step.
    g = torch.Generator().manual_seed(2)
    x = torch.randn(64, 4, 128, generator=g).to(torch.float16)
    q, s = quantize_int4_groupwise(x, group_size=32)
    amax = x.float().view(64, 4, 4, 32).abs().amax(-1)
    assert torch.equal(s, (amax / 7.0).clamp_min(2.0 ** -14).to(torch.float16))
    recon = q.float().view(64, 4, 4, 32) * s.float()[..., None]
    assert torch.all((recon - x.float().view(64, 4, 4, 32)).abs() <= s.float()[..., None] / 2 + 1e-7)
    assert int(q.abs().max()) <= 7


# ------------------------------------------------------- pack / unpack KATs
def test_pack_known_values():
    # test_correctness.py:85-101
    kat = GOLDEN["pack"]
    packed = pack_int4(torch.tensor([kat["q"]], dtype=torch.int8))
    assert packed.dtype == torch.uint8
    assert packed.flatten().tolist() == kat["packed"]


def test_pack_rejects_out_of_range():
    with pytest.raises(ValueError):
        pack_int4(torch.tensor([[-8, 0]], dtype=torch.int8))


def test_unpack_exhaustive_and_round_trip():
    b = torch.arange(256, dtype=torch.uint8)
    u = unpack_int4(b.view(256, 1)).view(256, 2).tolist()
    for byte, (lo, hi) in enumerate(u):
        nl, nh = byte & 0xF, byte >> 4
        assert lo == (nl - 16 if nl >= 8 else nl)  # nibble 8 decodes to -8
        assert hi == (nh - 16 if nh >= 8 else nh)
    q = torch.tensor([[a, c] for a in range(-7, 8) for c in range(-7, 8)], dtype=torch.int8)
    assert torch.equal(unpack_int4(pack_int4(q)), q)


def test_dequantize_closed_form():
    g = torch.Generator().manual_seed(3)
    packed = torch.randint(0, 256, (5, 3, 64), dtype=torch.uint8, generator=g)
    scales = torch.randn(5, 3, 4, generator=g).to(torch.float16)
    got = dequantize_int4_groupwise(packed, scales, group_size=32, dtype=torch.float32)
    q = unpack_int4(packed).float()
    want = q * scales.float().repeat_interleave(32, dim=-1)
    assert torch.equal(got, want)


# ---------------------------------------------------- append scenarios (KAT)
def _append_case():
    # test_correctness.py:104-183: T=4, Hkv=2, D=8, P=2, NP=4, group 4,
    # slots [3, 0, -1, 6], cos=1, sin=0.
    torch.manual_seed(3407)
    key = torch.randn(4, 2, 8, dtype=torch.float16)
    value = torch.rand_like(key)
    return {
        "key": key, "value": value,
        "positions": torch.tensor([0, 1, 2, 3], dtype=torch.int64),
        "slot_mapping": torch.tensor(GOLDEN["scattered_slots"], dtype=torch.int64),
        "cos_cache": torch.ones(4, 4, dtype=torch.float16),
        "sin_cache": torch.zeros(4, 4, dtype=torch.float16),
        "k_data": torch.randint(0, 256, (4, 2, 2, 4), dtype=torch.uint8),
        "v_data": torch.randint(0, 256, (4, 2, 2, 4), dtype=torch.uint8),
        "k_scale": torch.randn(4, 2, 2, 2, dtype=torch.float16),
        "v_scale": torch.randn(4, 2, 2, 2, dtype=torch.float16),
        "rotary_dim": 8, "group_size": 4, "page_size": 2,
    }


def _clone(case):
    return {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}


@pytest.mark.parametrize("impl", ["torch", "c"])
def test_append_scattered_slots(impl):
    # test_correctness.py:186-228
    case = _append_case()
    (torch_eager_append(**case) if impl == "torch" else c_append(case))
    valid = case["slot_mapping"] >= 0
    slots = case["slot_mapping"][valid]
    pages, offs = slots // 2, slots % 2
    kq, ks = quantize_int4_groupwise(case["key"][valid], group_size=4)
    vq, vs = quantize_int4_groupwise(case["value"][valid], group_size=4)
    assert torch.equal(case["k_data"][pages, offs], pack_int4(kq))
    assert torch.equal(case["v_data"][pages, offs], pack_int4(vq))
    assert torch.equal(case["k_scale"][pages, offs], ks)
    assert torch.equal(case["v_scale"][pages, offs], vs)


@pytest.mark.parametrize("impl", ["torch", "c"])
def test_append_leaves_other_slots_untouched(impl):
    # test_correctness.py:231-271
    case = _append_case()
    before = _clone(case)
    (torch_eager_append(**case) if impl == "torch" else c_append(case))
    mask = torch.zeros(4, 2, dtype=torch.bool)
    s = case["slot_mapping"][case["slot_mapping"] >= 0]
    mask[s // 2, s % 2] = True
    for name in ("k_data", "v_data", "k_scale", "v_scale"):
        assert torch.equal(case[name][~mask], before[name][~mask])


@pytest.mark.parametrize("impl", ["torch", "c"])
def test_append_all_negative_slots_is_noop(impl):
    # test_correctness.py:274-292
    case = _append_case()
    case["slot_mapping"] = torch.full_like(case["slot_mapping"], -1)
    before = _clone(case)
    (torch_eager_append(**case) if impl == "torch" else c_append(case))
    for name in ("k_data", "v_data", "k_scale", "v_scale"):
        assert torch.equal(case[name], before[name])


@pytest.mark.parametrize("impl", ["torch", "c"])
def test_append_rejects_duplicate_slots(impl):
    # test_correctness.py:295-305
    case = _append_case()
    case["slot_mapping"] = torch.tensor([3, 0, 3, 6], dtype=torch.int64)
    with pytest.raises(ValueError):
        (torch_eager_append(**case) if impl == "torch" else c_append(case))


@pytest.mark.parametrize("impl", ["torch", "c"])
@pytest.mark.parametrize("field,value,exc", [
    ("positions", [0, -1, 2, 3], IndexError),
    ("positions", [0, 1, 2, 4], IndexError),
    ("slot_mapping", [3, 0, -1, 8], IndexError),
])
def test_append_range_errors(impl, field, value, exc):
    # torch_eager_kv.py:290-305
    case = _append_case()
    case[field] = torch.tensor(value, dtype=torch.int64)
    with pytest.raises(exc):
        (torch_eager_append(**case) if impl == "torch" else c_append(case))


def test_append_torch_and_c_agree_on_kat_case():
    a, b = _append_case(), _append_case()
    torch_eager_append(**a)
    c_append(b)
    for name in ("k_data", "v_data", "k_scale", "v_scale"):
        assert torch.equal(a[name].view(torch.uint8), b[name].view(torch.uint8))


def test_quantize_non_finite_groups_follow_torch():
    # torch_eager_kv.py:69-86 on non-finite input: amax and clamp_min keep
    # NaN, so a NaN group's scale is NaN (stored by torch as 0x7E00 whatever
    # the payload) and an infinite group's is inf; x / scale is then +-0 or
    # NaN, which round/clamp keep and float -> int8 turns into 0.  Pinned
    # against torch's own ops on plain tensors, not against the oracle's code.
    from oracle.torch_eager_kv import quantize_int4_groupwise

    x = torch.randn(4, 64).to(torch.float16)
    x[0, 3] = float("nan")
    x[1, 40] = float("inf")
    x[2, 0] = -float("inf")
    x[2, 1] = float("nan")
    x[3, 33] = torch.tensor(0x7D01, dtype=torch.int16).view(torch.float16)  # a signalling-NaN payload
    q, s = quantize_int4_groupwise(x, 32)
    sb = s.view(torch.int16)
    assert sb[0, 0].item() == 0x7E00 and sb[1, 1].item() == 0x7C00
    assert sb[2, 0].item() == 0x7E00 and sb[3, 1].item() == 0x7E00
    assert not q[0, :32].any() and not q[1, 32:].any() and not q[2, :32].any() and not q[3, 32:].any()
    # the finite groups are untouched by their neighbours
    assert torch.isfinite(s[0, 1].float()) and torch.isfinite(s[1, 0].float())
    # the same values straight from torch's ops
    nan_group = torch.full((32,), float("nan"))
    assert torch.round(nan_group / nan_group).clamp(-7, 7).to(torch.int8).eq(0).all()
    assert (nan_group.abs().amax() / 7.0).clamp_min(2.0 ** -14).to(torch.float16).view(torch.int16).item() == 0x7E00
