"""Fused RoPE + INT4 append on the GPU: bit-exact against the checker
(oracle.torch_eager_kv, a restatement of the reference's torch_eager_append)
and the reference wrapper's error behaviour.  Packed bytes AND fp16 scales
must be identical (the reference test allows 2e-3 on k_scale; this does not)."""
import json
from pathlib import Path

import pytest
import torch

from helpers import KW, log, to
from iris_kernel import workloads
from iris_kernel.fused_kv import _rope_int4_paged_append, fused_rope_int4_paged_append
from oracle.torch_eager_kv import torch_eager_append

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def run_both(device, key, value, pos, slots, cos, sin, cache, rotary_dim):
    ref = tuple(t.clone() for t in cache)
    gpu = to(device, *cache)
    torch_eager_append(key, value, pos, slots, cos, sin, *ref, rotary_dim=rotary_dim, **KW)
    fused_rope_int4_paged_append(*to(device, key, value, pos, slots, cos, sin), *gpu,
                                 rotary_dim=rotary_dim, **KW)
    torch.cuda.synchronize(device)
    return ref, gpu


def assert_same(ref, gpu):
    for name, a, b in zip(("k_data", "v_data", "k_scale", "v_scale"), ref, gpu):
        a8, b8 = a.view(torch.uint8), b.cpu().view(torch.uint8)
        n_bad = int((a8 != b8).sum())
        assert n_bad == 0, f"{name}: {n_bad} bytes differ"


def test_reference_fused_append_scenario(device):
    # test_correctness.py:592-748: T=7, Hkv=4, D=128, P=16, NP=4,
    # slots [17, 2, -1, 31, 32, 47, 63], caches pre-filled with random bytes.
    log("append: reference scenario")
    g = torch.Generator().manual_seed(3407)
    T, H, D, NP = 7, 4, 128, 4
    key = torch.randn(T, H, D, generator=g).to(torch.float16)
    value = torch.randn(T, H, D, generator=g).to(torch.float16)
    pos = torch.arange(T, dtype=torch.int32)
    slots = torch.tensor(GOLDEN["fused_append_slots"], dtype=torch.int32)
    cos, sin = workloads.make_rope_cache(T, D)
    cache = (torch.randint(0, 256, (NP, 16, H, D // 2), dtype=torch.uint8, generator=g),
             torch.randint(0, 256, (NP, 16, H, D // 2), dtype=torch.uint8, generator=g),
             torch.randn(NP, 16, H, D // 32, generator=g).to(torch.float16),
             torch.randn(NP, 16, H, D // 32, generator=g).to(torch.float16))
    ref, gpu = run_both(device, key, value, pos, slots, cos, sin, cache, D)
    assert_same(ref, gpu)


@pytest.mark.parametrize("cfg", [1, 2, 4, 5])
def test_config_append_bit_exact(device, cfg):
    case = workloads.append_case(cfg)
    log(f"append: config {cfg}, T={case.key.shape[0]}")
    cache = case.empty_cache(fill="random")
    ref, gpu = run_both(device, case.key, case.value, case.positions, case.slot_mapping, case.cos,
                        case.sin, cache, case.config.head_dim)
    assert_same(ref, gpu)


@pytest.mark.parametrize("head_dim,page_size", [(64, 16), (128, 16), (192, 16), (256, 16), (512, 16),
                                                (32, 16), (96, 16), (160, 16), (224, 16), (480, 16),
                                                (96, 1), (96, 48), (128, 8), (320, 48)])
def test_head_dims_and_skipped_slots(device, head_dim, page_size):
    # head dims that are multiples of 32 up to 512 (192 and 96 exercise
    # padded lanes; an odd number of 32-dim groups -- 32, 96, 160, 224, 480 --
    # stores each scale on its own, rows being 2-byte aligned), page sizes
    # other than 16, an odd number of kv heads, random non-contiguous slots
    # with skips
    log(f"append: head_dim {head_dim} page_size {page_size}")
    g = torch.Generator().manual_seed(head_dim + page_size)
    T, H, NP = 37, 3, -(-96 // page_size)
    P = page_size
    key = (torch.randn(T, H, head_dim, generator=g) * 3).to(torch.float16)
    value = torch.randn(T, H, head_dim, generator=g).to(torch.float16)
    pos = torch.randint(0, 50, (T,), generator=g, dtype=torch.int32)
    slots = torch.randperm(NP * P, generator=g)[:T].to(torch.int32)
    slots[::5] = -1
    cos, sin = workloads.make_rope_cache(50, head_dim)
    cache = (torch.zeros(NP, P, H, head_dim // 2, dtype=torch.uint8),
             torch.zeros(NP, P, H, head_dim // 2, dtype=torch.uint8),
             torch.full((NP, P, H, head_dim // 32), -1.0, dtype=torch.float16),
             torch.full((NP, P, H, head_dim // 32), -1.0, dtype=torch.float16))
    ref = tuple(t.clone() for t in cache)
    gpu = to(device, *cache)
    torch_eager_append(key, value, pos, slots, cos, sin, *ref, rotary_dim=head_dim, group_size=32, page_size=P)
    fused_rope_int4_paged_append(*to(device, key, value, pos, slots, cos, sin), *gpu, rotary_dim=head_dim,
                                 group_size=32, page_size=P)
    torch.cuda.synchronize(device)
    assert_same(ref, gpu)


@pytest.mark.parametrize("head_dim", [80, 544])
def test_unsupported_head_dim_raises(device, head_dim):
    # a multiple of the 32-dim group up to 512, else NotImplementedError
    x = torch.zeros(2, 1, head_dim, dtype=torch.float16, device=device)
    i = torch.zeros(2, dtype=torch.int32, device=device)
    cache = (torch.zeros(1, 16, 1, head_dim // 2, dtype=torch.uint8, device=device),) * 2 + \
            (torch.zeros(1, 16, 1, head_dim // 32, dtype=torch.float16, device=device),) * 2
    cs = torch.zeros(4, head_dim // 2, dtype=torch.float16, device=device)
    with pytest.raises(NotImplementedError):
        fused_rope_int4_paged_append(x, x, i, i, cs, cs, *cache, rotary_dim=head_dim, group_size=32, page_size=16)


def test_ties_subnormals_and_extremes(device):
    # exact half-way quotients, fp16 subnormals, zero groups and |x| up to 3e4
    # (finite inputs: an inf makes the reference scale inf, outside the format)
    log("append: ties / subnormals / extremes")
    g = torch.Generator().manual_seed(17)
    T, H, D = 256, 2, 128
    base = torch.randint(-14, 15, (T, H, D), generator=g).float() / 2
    mult = torch.tensor([1.0, 0.5, 2.0 ** -14, 3.0, 1000.0])[torch.randint(0, 5, (T, H, 1), generator=g)]
    key = (base * mult).to(torch.float16)
    key[::7, :, :32] = 0  # zero groups
    value = (torch.randn(T, H, D, generator=g).clamp(-6, 6) * torch.tensor([1e-6, 1e-3, 1.0, 5e3])[
        torch.randint(0, 4, (T, 1, 1), generator=g)]).to(torch.float16)
    value[:, :, 5] = (torch.randint(-7, 8, (T, H), generator=g).float() + 0.5).to(torch.float16)
    pos = torch.randint(0, 64, (T,), generator=g, dtype=torch.int32)
    slots = torch.randperm(T * 2, generator=g)[:T].to(torch.int32)
    cos, sin = workloads.make_rope_cache(64, D)
    cache = tuple(t.to(torch.uint8) if i < 2 else t for i, t in enumerate(
        (torch.zeros(32, 16, H, D // 2), torch.zeros(32, 16, H, D // 2),
         torch.zeros(32, 16, H, D // 32, dtype=torch.float16), torch.zeros(32, 16, H, D // 32, dtype=torch.float16))))
    ref, gpu = run_both(device, key, value, pos, slots, cos, sin, cache, D)
    assert_same(ref, gpu)


def test_nan_and_inf_rows(device):
    # torch.amax and clamp_min propagate NaN: a group holding a NaN gets the
    # scale 0x7E00 (torch's fp16 NaN), one holding an infinity 0x7C00, and
    # every code of such a group is 0 (x / scale is +-0 or NaN, and float ->
    # int8 gives 0).  RoPE turns an infinite K next to a zero sine into NaN
    # (inf * 0), so K rows at position 0 exercise that path too.
    log("append: NaN / inf rows")
    g = torch.Generator().manual_seed(23)
    T, H, D = 48, 4, 128
    key = torch.randn(T, H, D, generator=g).to(torch.float16)
    value = torch.randn(T, H, D, generator=g).to(torch.float16)
    nan, inf = float("nan"), float("inf")
    key[0, 0, 3] = nan
    key[1, 1, 70] = inf
    key[2, 2, 100] = -inf
    key[3, 3, 5] = inf
    key[3, 3, 37] = nan
    value[4, 0, 31] = nan
    value[5, 1, 64] = -inf
    value[6, 2, :] = inf
    value[7, 3, 96:] = nan
    key[8:16] = nan
    value[16:24, :, 32:64] = -inf
    pos = torch.randint(0, 40, (T,), generator=g, dtype=torch.int32)
    pos[1:4] = 0  # sin = 0: inf * 0 = NaN in the rotated partner dims
    slots = torch.randperm(4 * 16, generator=g)[:T].to(torch.int32)
    cos, sin = workloads.make_rope_cache(40, D)
    cache = (torch.randint(0, 256, (4, 16, H, D // 2), dtype=torch.uint8, generator=g),
             torch.randint(0, 256, (4, 16, H, D // 2), dtype=torch.uint8, generator=g),
             torch.randn(4, 16, H, D // 32, generator=g).to(torch.float16),
             torch.randn(4, 16, H, D // 32, generator=g).to(torch.float16))
    ref, gpu = run_both(device, key, value, pos, slots, cos, sin, cache, D)
    # the case really has non-finite groups on both sides
    ks = ref[2].view(torch.int16)
    assert (ks == 0x7E00).any() and (ref[3].view(torch.int16) == 0x7C00).any()
    assert_same(ref, gpu)


def test_private_positional_handle(device):
    case = workloads.append_case(2)
    cache = case.empty_cache(fill="random")
    ref = tuple(t.clone() for t in cache)
    torch_eager_append(case.key, case.value, case.positions, case.slot_mapping, case.cos, case.sin,
                       *ref, rotary_dim=128, **KW)
    gpu = to(device, *cache)
    _rope_int4_paged_append(*to(device, case.key, case.value, case.positions, case.slot_mapping,
                                case.cos, case.sin), *gpu, 128, 16, 64)
    torch.cuda.synchronize(device)
    assert_same(ref, gpu)


def _small(device):
    g = torch.Generator().manual_seed(1)
    T, H, D, NP = 4, 2, 64, 2
    t = dict(key=torch.randn(T, H, D, generator=g).to(torch.float16),
             value=torch.randn(T, H, D, generator=g).to(torch.float16),
             positions=torch.arange(T, dtype=torch.int32),
             slot_mapping=torch.tensor([0, 5, -1, 9], dtype=torch.int32),
             cos_cache=torch.ones(8, D // 2, dtype=torch.float16),
             sin_cache=torch.zeros(8, D // 2, dtype=torch.float16),
             k_data=torch.zeros(NP, 16, H, D // 2, dtype=torch.uint8),
             v_data=torch.zeros(NP, 16, H, D // 2, dtype=torch.uint8),
             k_scale=torch.zeros(NP, 16, H, D // 32, dtype=torch.float16),
             v_scale=torch.zeros(NP, 16, H, D // 32, dtype=torch.float16))
    return {k: v.to(device) for k, v in t.items()}


@pytest.mark.parametrize("mutate,exc", [
    (lambda a, kw: a.update(slot_mapping=torch.tensor([0, 5, 5, 9], dtype=torch.int32, device=a["key"].device)), ValueError),
    (lambda a, kw: a.update(slot_mapping=torch.tensor([0, 5, -1, 32], dtype=torch.int32, device=a["key"].device)), IndexError),
    (lambda a, kw: a.update(positions=torch.tensor([0, -1, 2, 3], dtype=torch.int32, device=a["key"].device)), IndexError),
    (lambda a, kw: a.update(positions=torch.tensor([0, 1, 2, 8], dtype=torch.int32, device=a["key"].device)), IndexError),
    (lambda a, kw: a.update(positions=a["positions"].long()), TypeError),
    (lambda a, kw: a.update(key=a["key"].float(), value=a["value"].float()), TypeError),
    (lambda a, kw: a.update(cos_cache=a["cos_cache"].float()), TypeError),
    (lambda a, kw: kw.update(group_size=16), NotImplementedError),
    (lambda a, kw: kw.update(rotary_dim=32), ValueError),   # cos/sin width 32 is not rotary_dim // 2
    (lambda a, kw: kw.update(rotary_dim=66), ValueError),
    (lambda a, kw: kw.update(rotary_dim=-2), ValueError),
    (lambda a, kw: kw.update(rotary_dim=63), ValueError),
    (lambda a, kw: a.update(k_data=a["k_data"][:, :8]), ValueError),
    (lambda a, kw: a.update(key=a["key"].cpu()), ValueError),
])
def test_validation_errors(device, mutate, exc):
    a = _small(device)
    kw = dict(rotary_dim=64, group_size=32, page_size=16)
    mutate(a, kw)
    with pytest.raises(exc):
        fused_rope_int4_paged_append(**a, **kw)


@pytest.mark.parametrize("head_dim,rotary_dim", [
    (128, 0), (128, 16), (128, 64), (128, 96), (128, 112),   # multiples of 16: vector RoPE path
    (128, 2), (128, 6), (128, 34), (128, 100), (128, 126),   # per-element path
    (64, 32), (64, 10), (256, 128), (256, 250), (512, 256),
    (96, 96), (96, 48), (96, 10), (32, 32), (32, 6), (160, 64), (480, 480)])
def test_partial_rotary_bit_exact(device, head_dim, rotary_dim):
    # Partial RoPE as the eager path defines it (torch_eager_kv.py:35-49):
    # the first rotary_dim dims rotate, the rest pass through.
    log(f"append: partial rotary D={head_dim} R={rotary_dim}")
    g = torch.Generator().manual_seed(head_dim * 1000 + rotary_dim)
    T, H, NP, P = 37, 3, 6, 16
    key = (torch.randn(T, H, head_dim, generator=g) * 3).to(torch.float16)
    value = (torch.randn(T, H, head_dim, generator=g) * 3).to(torch.float16)
    pos = torch.randint(0, 500, (T,), generator=g, dtype=torch.int32)
    slots = torch.randperm(NP * P, generator=g)[:T].to(torch.int32)
    slots[::7] = -1
    ang = torch.rand(500, rotary_dim // 2, generator=g) * 300
    cos, sin = ang.cos().to(torch.float16), ang.sin().to(torch.float16)
    cache = (torch.randint(0, 256, (NP, P, H, head_dim // 2), dtype=torch.uint8, generator=g),
             torch.randint(0, 256, (NP, P, H, head_dim // 2), dtype=torch.uint8, generator=g),
             torch.randn(NP, P, H, head_dim // 32, generator=g).to(torch.float16),
             torch.randn(NP, P, H, head_dim // 32, generator=g).to(torch.float16))
    ref, gpu = run_both(device, key, value, pos, slots, cos, sin, cache, rotary_dim)
    assert_same(ref, gpu)


def test_invalid_slot_positions_are_not_read(device):
    # positions of skipped tokens may be anything (fused_kv.py:741-759 only
    # checks valid tokens): the kernel must neither read them nor write.
    a = _small(device)
    a["slot_mapping"] = torch.tensor([-1, 5, -1, -1], dtype=torch.int32, device=device)
    a["positions"] = torch.tensor([10 ** 9, 1, -(10 ** 9), 7], dtype=torch.int32, device=device)
    before = [a[n].clone() for n in ("k_data", "v_data", "k_scale", "v_scale")]
    fused_rope_int4_paged_append(**a, rotary_dim=64, group_size=32, page_size=16)
    torch.cuda.synchronize(device)
    changed = (a["k_data"] != before[0]).any(dim=(2, 3))
    assert changed.nonzero().tolist() == [[0, 5]]


def test_all_negative_slots_is_noop(device):
    a = _small(device)
    a["slot_mapping"].fill_(-1)
    before = [a[n].clone() for n in ("k_data", "v_data", "k_scale", "v_scale")]
    fused_rope_int4_paged_append(**a, rotary_dim=64, group_size=32, page_size=16)
    torch.cuda.synchronize(device)
    for n, b in zip(("k_data", "v_data", "k_scale", "v_scale"), before):
        assert torch.equal(a[n], b)
