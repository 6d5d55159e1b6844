"""The fp16-cache RoPE append and the standalone INT4 quantise-pack on the GPU,
through the C ABI, bit-exact against the checker (apply_rope,
quantize_int4_groupwise, pack_int4 of oracle/torch_eager_kv.py): the
reference's own scenarios (tests/test_correctness.py:330-592), partial
rotary_dim on both kernel paths, untouched cache regions, the benchmark
append workloads, fp16 edge values and the reference's exception types."""
import pytest
import torch

from helpers import log, to
from iris_kernel import workloads
from iris_kernel.fused_kv import (_quantize_pack_int4_g32, _rope_fp16_paged_append, fused_quantize_pack_int4,
                                  fused_rope_fp16_append)
from oracle.torch_eager_kv import apply_rope, pack_int4, quantize_int4_groupwise

pytestmark = pytest.mark.gpu


def expected_fp16_cache(key, value, positions, slots, cos, sin, k_cache, v_cache, rotary_dim, page_size=16):
    """The checker: RoPE(K) by apply_rope (fp16, every op rounded) and V at
    the valid slots of copies of the caches."""
    ek, ev = k_cache.clone(), v_cache.clone()
    valid = slots >= 0
    s = slots[valid].long()
    pos = positions[valid].long()
    rk = apply_rope(key[valid], cos[pos][:, None, :], sin[pos][:, None, :], rotary_dim=rotary_dim)
    ek[s // page_size, s % page_size] = rk
    ev[s // page_size, s % page_size] = value[valid]
    return ek, ev


def run_fp16_append(device, key, value, positions, slots, cos, sin, k_cache, v_cache, rotary_dim, page_size=16):
    kc, vc = to(device, k_cache, v_cache)
    fused_rope_fp16_append(*to(device, key, value, positions, slots, cos, sin), kc, vc, rotary_dim=rotary_dim,
                           page_size=page_size)
    torch.cuda.synchronize(device)
    return kc.cpu(), vc.cpu()


def assert_bits(got, want, what):
    g, w = got.view(torch.int16), want.view(torch.int16)
    bad = (g != w).sum().item()
    assert bad == 0, f"{what}: {bad} fp16 values differ from the checker"


def test_fp16_append_reference_scenario(device):
    # test_correctness.py:330-462: 7 tokens, Hkv=4, D=128, slots
    # [17, 2, -1, 31, 32, 47, 63] over 4 pages of random cache.
    torch.manual_seed(3407)
    T, H, D, P, NP = 7, 4, 128, 16, 4
    key = torch.randn(T, H, D, dtype=torch.float16)
    value = torch.randn_like(key)
    positions = torch.arange(T, dtype=torch.int32)
    slots = torch.tensor([17, 2, -1, 31, 32, 47, 63], dtype=torch.int32)
    cos, sin = workloads.make_rope_cache(T, D)
    kc = torch.randn(NP, P, H, D, dtype=torch.float16)
    vc = torch.randn_like(kc)
    ek, ev = expected_fp16_cache(key, value, positions, slots, cos, sin, kc, vc, D)
    gk, gv = run_fp16_append(device, key, value, positions, slots, cos, sin, kc, vc, D)
    assert_bits(gk, ek, "k_cache")
    assert torch.equal(gv, ev)


@pytest.mark.parametrize("d,rot", [(128, 128), (128, 64), (128, 32), (128, 0), (64, 48), (72, 16), (36, 12),
                                   (128, 2), (256, 256), (96, 80)])
def test_fp16_append_partial_rotary_dims(device, d, rot):
    # rot % 16 == 0 with d % 8 == 0 runs the 16-byte-per-lane kernel, the
    # rest the one-element kernel; both must match apply_rope bit for bit,
    # and cache rows that no token writes must not change.
    g = torch.Generator().manual_seed(d * 1000 + rot)
    T, H, P, NP = 37, 3, 16, 6
    key = (torch.randn(T, H, d, generator=g) * 3).to(torch.float16)
    value = torch.randn(T, H, d, generator=g).to(torch.float16)
    positions = torch.randint(0, 500, (T,), generator=g, dtype=torch.int32)
    slots = torch.randperm(NP * P, generator=g)[:T].to(torch.int32)
    slots[::5] = -1
    cos, sin = workloads.make_rope_cache(500, rot) if rot else (torch.zeros(500, 0, dtype=torch.float16),) * 2
    kc = torch.randn(NP, P, H, d, generator=g).to(torch.float16)
    vc = torch.randn(NP, P, H, d, generator=g).to(torch.float16)
    ek, ev = expected_fp16_cache(key, value, positions, slots, cos, sin, kc, vc, rot)
    gk, gv = run_fp16_append(device, key, value, positions, slots, cos, sin, kc, vc, rot)
    assert_bits(gk, ek, f"k_cache d={d} rot={rot}")
    assert torch.equal(gv, ev)


@pytest.mark.parametrize("cfg", [1, 2, 4, 5])
def test_fp16_append_config_workloads(device, cfg):
    case = workloads.append_case(cfg)
    c = case.config
    kc = torch.zeros(case.num_pages, 16, c.num_kv_heads, c.head_dim, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    ek, ev = expected_fp16_cache(case.key, case.value, case.positions, case.slot_mapping, case.cos, case.sin,
                                 kc, vc, c.head_dim)
    gk, gv = run_fp16_append(device, case.key, case.value, case.positions, case.slot_mapping, case.cos,
                             case.sin, kc, vc, c.head_dim)
    assert_bits(gk, ek, f"cfg{cfg} k_cache")
    assert torch.equal(gv, ev)
    log(f"fp16 append: config {cfg} ({case.key.shape[0]} tokens) bit-exact")


def test_fp16_append_private_handle(device):
    case = workloads.append_case(1)
    c = case.config
    kc = torch.zeros(case.num_pages, 16, c.num_kv_heads, c.head_dim, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    ek, ev = expected_fp16_cache(case.key, case.value, case.positions, case.slot_mapping, case.cos, case.sin,
                                 kc, vc, c.head_dim)
    gk, gv = to(device, kc, vc)
    _rope_fp16_paged_append(*to(device, case.key, case.value, case.positions, case.slot_mapping, case.cos,
                                case.sin), gk, gv, c.head_dim, c.head_dim, 16, 64)
    torch.cuda.synchronize(device)
    assert_bits(gk.cpu(), ek, "private handle k_cache")
    assert torch.equal(gv.cpu(), ev)


def test_fp16_append_validation_errors(device):
    # fused_kv.py:166-282: the reference's exception types, in its order.
    T, H, D = 4, 2, 64
    key = torch.randn(T, H, D, dtype=torch.float16, device=device)
    pos = torch.arange(T, dtype=torch.int32, device=device)
    slots = torch.arange(T, dtype=torch.int32, device=device)
    cos, sin = to(device, *workloads.make_rope_cache(8, D))
    kc = torch.zeros(2, 16, H, D, dtype=torch.float16, device=device)
    vc = torch.zeros_like(kc)

    def call(**kw):
        a = dict(key=key, value=key, positions=pos, slot_mapping=slots, cos_cache=cos, sin_cache=sin,
                 k_cache=kc, v_cache=vc)
        extra = {k: kw.pop(k) for k in ("rotary_dim", "page_size") if k in kw}
        a.update(kw)
        fused_rope_fp16_append(a["key"], a["value"], a["positions"], a["slot_mapping"], a["cos_cache"],
                               a["sin_cache"], a["k_cache"], a["v_cache"], rotary_dim=extra.get("rotary_dim", D),
                               page_size=extra.get("page_size", 16))

    with pytest.raises(ValueError):
        call(key=key.cpu())
    with pytest.raises(ValueError):
        call(value=key[:2])
    with pytest.raises(TypeError):
        call(key=key.float(), value=key.float())
    with pytest.raises(ValueError):
        call(rotary_dim=D + 2)
    with pytest.raises(ValueError):
        call(rotary_dim=3)
    with pytest.raises(ValueError):
        call(k_cache=kc[..., :32])
    with pytest.raises(TypeError):
        call(k_cache=kc.float(), v_cache=vc.float())
    with pytest.raises(TypeError):
        call(positions=pos.long())
    with pytest.raises(ValueError):
        call(cos_cache=cos[:, :8], sin_cache=sin[:, :8])
    with pytest.raises(TypeError):
        call(cos_cache=cos.float(), sin_cache=sin.float())
    dup = slots.clone()
    dup[1] = dup[0]
    with pytest.raises(ValueError, match="duplicate"):
        call(slot_mapping=dup)
    with pytest.raises(IndexError):
        call(slot_mapping=slots + 32)
    with pytest.raises(IndexError):
        call(positions=pos + 8)
    neg = pos.clone()
    neg[0] = -1
    with pytest.raises(IndexError):
        call(positions=neg)
    # every slot skipped: a no-op, whatever the positions
    call(slot_mapping=torch.full_like(slots, -1), positions=pos + 100)
    assert not kc.any()


def _edge_values(d: int) -> torch.Tensor:
    """[T, 3, d] fp16 rows that stress the quantiser: zero groups, exact
    ties x / s = k + 1/2, subnormals, +-65504, single large outliers."""
    g = torch.Generator().manual_seed(d)
    rows = [torch.zeros(d), torch.full((d,), 65504.0), torch.full((d,), -65504.0),
            torch.full((d,), 2.0 ** -24), torch.linspace(-7.5, 7.5, d)]
    x = torch.randn(d, generator=g)
    x[::32] = 300.0
    rows.append(x)
    for k in range(8):  # scale 1.0 (amax 7) with every tie k + 1/2
        r = torch.full((d,), k + 0.5)
        r[::32] = 7.0
        rows.append(r)
    t = torch.stack(rows).to(torch.float16)
    return torch.stack([t, -t, t * 0.001], dim=1)


def _non_finite_rows(d):
    # NaN / +-inf in single dims, whole groups and whole rows: the group's
    # scale becomes 0x7E00 (NaN) or 0x7C00 (inf) and its codes 0, as
    # torch.amax / clamp_min / float->int8 give them.
    g = torch.Generator().manual_seed(d)
    x = torch.randn(16, 3, d, generator=g).to(torch.float16)
    nan, inf = float("nan"), float("inf")
    x[0, 0, 1] = nan
    x[1, 1, d - 1] = inf
    x[2, 2, 33 % d] = -inf
    x[3, 0, 0] = inf
    x[3, 0, 1] = nan
    x[4, :, :32] = nan
    x[5, 1, :] = -inf
    x[6] = nan
    return x


@pytest.mark.parametrize("head_dim", [64, 128, 256, 512])
def test_quantize_pack_matches_eager(device, head_dim):
    # test_correctness.py:465-592 (head_dim 64, 128, 256; 7 x 4 random
    # rows), plus 512 and the edge rows: packed bytes and scales bit-exact.
    torch.manual_seed(3407)
    for name, x in (("random", torch.randn(7, 4, head_dim, dtype=torch.float16)),
                    ("edges", _edge_values(head_dim)),
                    ("bulk", (torch.randn(4096, 8, head_dim) * 4).to(torch.float16)),
                    ("non-finite", _non_finite_rows(head_dim))):
        q_ref, s_ref = quantize_int4_groupwise(x, group_size=32)
        p_ref = pack_int4(q_ref)
        xg = x.to(device)
        packed = torch.empty(p_ref.shape, dtype=torch.uint8, device=device)
        scales = torch.empty(s_ref.shape, dtype=torch.float16, device=device)
        fused_quantize_pack_int4(xg, packed, scales)
        torch.cuda.synchronize(device)
        assert torch.equal(packed.cpu(), p_ref), f"{name} d={head_dim}: packed bytes differ"
        assert torch.equal(scales.cpu().view(torch.int16), s_ref.view(torch.int16)), f"{name}: scales differ"
    out_p = torch.empty(p_ref.shape, dtype=torch.uint8, device=device)
    out_s = torch.empty(s_ref.shape, dtype=torch.float16, device=device)
    _quantize_pack_int4_g32(xg, out_p, out_s, head_dim, 64)
    torch.cuda.synchronize(device)
    assert torch.equal(out_p.cpu(), p_ref)


def test_quantize_pack_validation_errors(device):
    x = torch.randn(3, 2, 128, dtype=torch.float16, device=device)
    p = torch.empty(3, 2, 64, dtype=torch.uint8, device=device)
    s = torch.empty(3, 2, 4, dtype=torch.float16, device=device)
    with pytest.raises(ValueError):
        fused_quantize_pack_int4(x.cpu(), p, s)
    with pytest.raises(ValueError):
        fused_quantize_pack_int4(x[0], p, s)
    with pytest.raises(TypeError):
        fused_quantize_pack_int4(x.float(), p, s)
    with pytest.raises(NotImplementedError):
        fused_quantize_pack_int4(x[..., :96], p[..., :48], s[..., :3])
    with pytest.raises(ValueError):
        fused_quantize_pack_int4(x, p[..., :32], s)
    with pytest.raises(ValueError):
        fused_quantize_pack_int4(x, p, s[..., :2])
    with pytest.raises(TypeError):
        fused_quantize_pack_int4(x, p.to(torch.int8), s)
    with pytest.raises(TypeError):
        fused_quantize_pack_int4(x, p, s.float())
    with pytest.raises(ValueError):
        fused_quantize_pack_int4(x, p.cpu(), s)
