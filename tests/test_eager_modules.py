"""The drop-in package's eager modules (iris_kernel.torch_eager_kv and
iris_kernel.torch_eager_attention, product code) pinned on the CPU against
the checkers under oracle/ and the reference's known answers: bit-exact for
RoPE, quantisation, packing, the append and unpacking; within fp32
reassociation for attention (the package batches sequences, the checker
loops over them); identical exceptions for invalid inputs.  Also: the
package modules import nothing from oracle/, and the reference's own import
lines resolve against the package."""
import json
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from iris_kernel import torch_eager_attention as pkg_attn
from iris_kernel import torch_eager_kv as pkg_kv
from oracle import torch_eager_attention as ora_attn
from oracle import torch_eager_kv as ora_kv

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_package_modules_import_nothing_from_oracle():
    code = ("import sys; import iris_kernel.torch_eager_kv, iris_kernel.torch_eager_attention; "
            "bad = [m for m in sys.modules if m == 'oracle' or m.startswith('oracle.')]; "
            "assert not bad, bad")
    env = {"PYTHONPATH": str(ROOT / "iris-kernel_amd"), "PATH": "/usr/bin:/bin"}
    subprocess.run([sys.executable, "-c", code], check=True, env=env, cwd="/")
    for mod in (pkg_kv, pkg_attn):
        text = Path(mod.__file__).read_text()
        assert "import oracle" not in text and "from oracle" not in text


def test_reference_import_lines_resolve():
    # tests/test_correctness.py:4-9 and tests/test_attention.py:9-13 of the reference
    from iris_kernel.torch_eager_attention import (  # noqa: F401
        torch_eager_fp16_paged_decode_attention, torch_eager_int4_paged_decode_attention)
    from iris_kernel.torch_eager_kv import apply_rope, pack_int4, quantize_int4_groupwise, torch_eager_append  # noqa: F401


# ------------------------------------------------------------ write side
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rotary_dim", [0, 32, 64])
def test_apply_rope_bit_exact(dtype, rotary_dim):
    g = torch.Generator().manual_seed(rotary_dim + 7)
    x = (torch.randn(9, 3, 64, generator=g) * 3).to(dtype)
    ang = torch.rand(9, 1, rotary_dim // 2, generator=g) * 20
    cos, sin = ang.cos().to(dtype), ang.sin().to(dtype)
    assert torch.equal(pkg_kv.apply_rope(x, cos, sin, rotary_dim), ora_kv.apply_rope(x, cos, sin, rotary_dim))


def test_rope_quarter_turn_kat():
    kat = GOLDEN["rope_quarter_turn"]
    out = pkg_kv.apply_rope(torch.tensor([[kat["x"]]]), torch.zeros(1, 1, 2), torch.ones(1, 1, 2), rotary_dim=4)
    torch.testing.assert_close(out, torch.tensor([[kat["expected"]]]))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("group_size", [8, 32, 64])
def test_quantize_and_pack_bit_exact(dtype, group_size):
    g = torch.Generator().manual_seed(group_size)
    x = (torch.randn(17, 4, 128, generator=g) * torch.rand(17, 4, 1, generator=g) * 10).to(dtype)
    x[0, 0, :group_size] = 0  # an all-zero group
    x[1, 1, 3] = float("nan")  # non-finite groups follow torch
    x[2, 2, 5] = float("inf")
    qp, sp = pkg_kv.quantize_int4_groupwise(x, group_size)
    qo, so = ora_kv.quantize_int4_groupwise(x, group_size)
    assert torch.equal(qp, qo)
    assert torch.equal(sp.view(torch.int16) if dtype != torch.float32 else sp.view(torch.int32),
                       so.view(torch.int16) if dtype != torch.float32 else so.view(torch.int32))
    assert torch.equal(pkg_kv.pack_int4(qp), ora_kv.pack_int4(qo))


def test_quantize_and_pack_kats():
    kat = GOLDEN["pack"]
    q = torch.tensor(kat["q"], dtype=torch.int8)
    assert pkg_kv.pack_int4(q).tolist() == kat["packed"]


def test_pack_and_quantize_errors_match():
    for bad in (torch.tensor([1, 8], dtype=torch.int8), torch.tensor([1, 2, 3], dtype=torch.int8),
                torch.tensor([1, 2], dtype=torch.int16)):
        with pytest.raises(Exception) as a:
            ora_kv.pack_int4(bad)
        with pytest.raises(type(a.value), match=str(a.value).replace("[", r"\[").replace("]", r"\]")):
            pkg_kv.pack_int4(bad)
    with pytest.raises(ValueError):
        pkg_kv.quantize_int4_groupwise(torch.zeros(2, 30), 32)


def _append_case(seed, dtype, n_tok, hkv, d, rotary_dim, group_size, page_size, n_pages, skip=0):
    g = torch.Generator().manual_seed(seed)
    key = (torch.randn(n_tok, hkv, d, generator=g) * 2).to(dtype)
    value = (torch.randn(n_tok, hkv, d, generator=g) * 2).to(dtype)
    positions = torch.randint(0, 300, (n_tok,), generator=g, dtype=torch.int32)
    slots = torch.randperm(n_pages * page_size, generator=g)[:n_tok].to(torch.int32)
    slots[:skip] = -1
    ang = torch.rand(300, rotary_dim // 2, generator=g) * 100
    cache = (torch.randint(0, 256, (n_pages, page_size, hkv, d // 2), generator=g, dtype=torch.uint8),
             torch.randint(0, 256, (n_pages, page_size, hkv, d // 2), generator=g, dtype=torch.uint8),
             torch.randn(n_pages, page_size, hkv, d // group_size, generator=g).to(dtype),
             torch.randn(n_pages, page_size, hkv, d // group_size, generator=g).to(dtype))
    return (key, value, positions, slots, ang.cos().to(dtype), ang.sin().to(dtype)), cache


@pytest.mark.parametrize("dtype,rotary_dim,group_size,page_size", [
    (torch.float16, 128, 32, 16), (torch.float16, 64, 32, 16), (torch.float16, 0, 64, 8),
    (torch.bfloat16, 96, 32, 32), (torch.float32, 128, 16, 16)])
def test_append_bit_exact(dtype, rotary_dim, group_size, page_size):
    args, cache = _append_case(3, dtype, 40, 4, 128, rotary_dim, group_size, page_size, 9, skip=5)
    mine = tuple(t.clone() for t in cache)
    want = tuple(t.clone() for t in cache)
    kw = dict(rotary_dim=rotary_dim, group_size=group_size, page_size=page_size)
    pkg_kv.torch_eager_append(*args, *mine, **kw)
    ora_kv.torch_eager_append(*args, *want, **kw)
    for a, b in zip(mine, want):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_append_errors_match():
    args, cache = _append_case(4, torch.float16, 8, 2, 64, 64, 32, 16, 2)
    key, value, positions, slots, cos, sin = args
    kw = dict(rotary_dim=64, group_size=32, page_size=16)
    dup = slots.clone()
    dup[1] = dup[0]
    far = slots.clone()
    far[2] = 10_000
    late = positions.clone()
    late[0] = 5000
    cases = [
        ((key, value[:, :1], positions, slots, cos, sin), kw),
        ((key, value.float(), positions, slots, cos, sin), kw),
        ((key, value, positions[:3], slots, cos, sin), kw),
        ((key, value, positions, slots, cos, sin), dict(kw, rotary_dim=3)),
        ((key, value, positions, slots, cos, sin), dict(kw, group_size=48)),
        ((key, value, positions, dup, cos, sin), kw),
        ((key, value, positions, far, cos, sin), kw),
        ((key, value, late, slots, cos, sin), kw),
        ((key, value, positions, slots, cos[:, :5], sin[:, :5]), kw),
    ]
    for a, k in cases:
        with pytest.raises(Exception) as want:
            ora_kv.torch_eager_append(*a, *cache, **k)
        with pytest.raises(type(want.value)) as got:
            pkg_kv.torch_eager_append(*a, *cache, **k)
        assert str(got.value) == str(want.value)


# ------------------------------------------------------------- read side
def test_unpack_every_byte():
    b = torch.arange(256, dtype=torch.uint8).reshape(16, 16)
    assert torch.equal(pkg_attn.unpack_int4(b), ora_attn.unpack_int4(b))


def test_dequantize_bit_exact():
    g = torch.Generator().manual_seed(9)
    packed = torch.randint(0, 256, (5, 3, 64), generator=g, dtype=torch.uint8)
    scales = torch.rand(5, 3, 4, generator=g).to(torch.float16)
    for dtype in (torch.float32, torch.float16):
        assert torch.equal(pkg_attn.dequantize_int4_groupwise(packed, scales, dtype=dtype),
                           ora_attn.dequantize_int4_groupwise(packed, scales, dtype=dtype))


def _decode_case(seed, batch, hq, hkv, d, lens, n_pages, page_size=16, table_dtype=torch.int32):
    g = torch.Generator().manual_seed(seed)
    max_pages = max(-(-n // page_size) for n in lens) + 1
    cache = (torch.randint(0, 256, (n_pages, page_size, hkv, d // 2), generator=g, dtype=torch.uint8),
             torch.randint(0, 256, (n_pages, page_size, hkv, d // 2), generator=g, dtype=torch.uint8),
             (torch.rand(n_pages, page_size, hkv, d // 32, generator=g) * 0.3).to(torch.float16),
             (torch.rand(n_pages, page_size, hkv, d // 32, generator=g) * 0.3).to(torch.float16))
    bt = torch.randint(0, n_pages, (batch, max_pages), generator=g).to(table_dtype)
    bt[:, -1] = -5  # never read: past every sequence's pages
    q = torch.randn(batch, hq, d, generator=g).to(torch.float16)
    return q, cache, bt, torch.tensor(lens, dtype=table_dtype)


@pytest.mark.parametrize("hq,hkv,d,lens,table_dtype", [
    (8, 2, 128, [1, 17, 300, 64], torch.int32),
    (32, 8, 128, [40, 513], torch.int64),
    (16, 1, 64, [7, 250, 33], torch.int32),
])
def test_int4_decode_matches_checker(hq, hkv, d, lens, table_dtype):
    q, cache, bt, sl = _decode_case(5, len(lens), hq, hkv, d, lens, 64, table_dtype=table_dtype)
    got = pkg_attn.torch_eager_int4_paged_decode_attention(q, *cache, bt, sl)
    want = ora_attn.torch_eager_int4_paged_decode_attention(q, *cache, bt, sl)
    assert got.dtype == torch.float16
    torch.testing.assert_close(got, want, atol=2e-3, rtol=0)
    s = pkg_attn.torch_eager_int4_paged_decode_attention(q, *cache, bt, sl, softmax_scale=0.05)
    torch.testing.assert_close(s, ora_attn.torch_eager_int4_paged_decode_attention(q, *cache, bt, sl,
                                                                                   softmax_scale=0.05),
                               atol=2e-3, rtol=0)


def test_int4_decode_reference_lengths_kat():
    lens = GOLDEN["attention_seq_lens"]
    lens = lens if isinstance(lens, list) else lens["seq_lens"]
    q, cache, bt, sl = _decode_case(6, len(lens), 8, 2, 64, lens, 64)
    torch.testing.assert_close(pkg_attn.torch_eager_int4_paged_decode_attention(q, *cache, bt, sl),
                               ora_attn.torch_eager_int4_paged_decode_attention(q, *cache, bt, sl),
                               atol=2e-3, rtol=0)


def test_fp16_decode_matches_checker():
    g = torch.Generator().manual_seed(8)
    lens = [5, 90, 200]
    kc = torch.randn(40, 16, 2, 64, generator=g).to(torch.float16)
    vc = torch.randn(40, 16, 2, 64, generator=g).to(torch.float16)
    bt = torch.randint(0, 40, (3, 14), generator=g).to(torch.int32)
    q = torch.randn(3, 8, 64, generator=g).to(torch.float16)
    sl = torch.tensor(lens, dtype=torch.int32)
    torch.testing.assert_close(pkg_attn.torch_eager_fp16_paged_decode_attention(q, kc, vc, bt, sl),
                               ora_attn.torch_eager_fp16_paged_decode_attention(q, kc, vc, bt, sl),
                               atol=2e-3, rtol=0)


def test_decode_errors_match():
    q, cache, bt, sl = _decode_case(7, 2, 8, 2, 64, [20, 40], 8)
    bad_ids = bt.clone()
    bad_ids[0, 0] = 99
    short = bt[:, :1]
    cases = [
        (q.float(), cache, bt, sl), (q[:, :3], cache, bt, sl), (q, cache, bad_ids, sl), (q, cache, short, sl),
        (q, cache, bt, torch.tensor([0, 3], dtype=torch.int32)), (q, cache, bt.to(torch.int16), sl),
        (q, (cache[0], cache[1], cache[2].float(), cache[3]), bt, sl),
    ]
    for qq, c, b, s in cases:
        with pytest.raises(Exception) as want:
            ora_attn.torch_eager_int4_paged_decode_attention(qq, *c, b, s)
        with pytest.raises(type(want.value)) as got:
            pkg_attn.torch_eager_int4_paged_decode_attention(qq, *c, b, s)
        assert str(got.value) == str(want.value)


def test_empty_batch_matches_reference_loop():
    """B = 0: the reference's per-sequence loops run zero times and return an
    empty [0, Hq, D] tensor (torch_eager_attention.py:188-239, :270-294);
    the package's batched forms return the same instead of reducing over an
    empty length tensor."""
    q, cache, bt, sl = _decode_case(9, 2, 8, 2, 64, [20, 40], 8)
    q0, bt0, sl0 = q[:0], bt[:0], sl[:0]
    got = pkg_attn.torch_eager_int4_paged_decode_attention(q0, *cache, bt0, sl0)
    want = ora_attn.torch_eager_int4_paged_decode_attention(q0, *cache, bt0, sl0)
    assert got.shape == want.shape == (0, 8, 64) and got.dtype == want.dtype == torch.float16
    kc = torch.zeros(4, 16, 2, 64, dtype=torch.float16)
    got16 = pkg_attn.torch_eager_fp16_paged_decode_attention(q0, kc, kc, bt0, sl0)
    want16 = ora_attn.torch_eager_fp16_paged_decode_attention(q0, kc, kc, bt0, sl0)
    assert got16.shape == want16.shape == (0, 8, 64) and got16.dtype == torch.float16
