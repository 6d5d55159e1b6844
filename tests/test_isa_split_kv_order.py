"""The split-KV arrival protocol in every decode kernel's compiled gfx950
code.  Partials travel between workgroups through device-coherent (sc1)
stores and loads, and the arrival is a relaxed agent-scope atomic
(arrive_last in csrc/common.h): the order rests on the code the compiler
emits.  For every arrival of every decode kernel: the partial stores before
it are complete (s_waitcnt vmcnt(0), then a workgroup barrier) before it is
issued, and the merge's first partial load after it is issued only after its
returned count has been waited for and broadcast (s_waitcnt vmcnt(0), then a
barrier).  Runs without a GPU."""
import pytest

from isa_hazards import kernel_lines, kernel_symbols, split_kv_order

DECODE_SOURCES = ["decode.hip", "decode_pages.hip", "decode_stream.hip", "decode_mqa.hip", "decode_fp16.hip",
                  "decode_fp16_stream.hip", "decode_any.hip", "decode_hd.hip"]


@pytest.mark.parametrize("src", DECODE_SOURCES)
def test_merges_read_partials_only_after_the_arrival(asm_by_source, src):
    asm = asm_by_source[src]
    checked = 0
    for sym in kernel_symbols(asm):
        bad, pairs = split_kv_order(kernel_lines(asm, sym))
        assert not bad, f"{src} {sym}: {bad[:3]}"
        checked += pairs
    assert checked > 0, f"{src}: no arrival followed by a merge load found"


def test_checker_flags_a_hoisted_merge_load_and_an_early_arrival():
    good = ["buffer_store_dwordx4 v[0:3], v4, s[8:11], 0 offen sc1",
            "s_waitcnt vmcnt(0)", "s_barrier",
            "global_atomic_add v3, v2, v3, s[10:11] sc0",
            "s_waitcnt vmcnt(0)", "ds_write_b32 v2, v3", "s_waitcnt lgkmcnt(0)", "s_barrier",
            "buffer_load_dwordx4 v[4:7], v5, s[8:11], 0 offen sc1"]
    assert split_kv_order(good) == ([], 1)
    hoisted = good[:4] + [good[-1]] + good[4:-1]   # the merge load right after the atomic
    bad, _ = split_kv_order(hoisted)
    assert len(bad) == 1 and "merge load" in bad[0]
    early = [good[0], good[3]] + good[4:]            # the arrival before the stores completed
    bad, _ = split_kv_order(early)
    assert len(bad) == 1 and "arrival" in bad[0]
