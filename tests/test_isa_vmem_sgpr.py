"""Every HIP source, compiled for gfx950: no vector-memory instruction reads
an SGPR that a VALU instruction wrote fewer than 5 wait states earlier (see
isa_hazards.vmem_sgpr_hazards).  The kernels issue some loads as inline
assembly, which the compiler does not pad; a descriptor restored with
v_readfirstlane right before such a load would address the wrong memory.
Uses the session's gfx950 assembly of every source; runs without a GPU."""
from isa_hazards import vmem_sgpr_hazards


def test_no_vmem_reads_an_sgpr_right_after_a_valu_write(asm_by_source):
    for src, asm in asm_by_source.items():
        bad = vmem_sgpr_hazards(asm.split("\n"))
        assert not bad, f"{src}: {bad[:5]}"


def test_checker_flags_a_descriptor_restored_by_readfirstlane():
    bad = ["v_readfirstlane_b32 s4, v24",
           "v_readfirstlane_b32 s5, v25",
           "buffer_load_dwordx4 v[18:21], v29, s[4:7], 0 offen nt"]
    load = "buffer_load_dwordx4 v[18:21], v29, s[4:7], 0 offen nt"
    assert vmem_sgpr_hazards(bad) == [(load, 1), (load, 0)]  # s4 one wait state back, s5 none
    padded = ["v_readfirstlane_b32 s4, v24",
              "s_nop 4",
              "buffer_load_dwordx4 v[18:21], v29, s[4:7], 0 offen nt"]
    assert vmem_sgpr_hazards(padded) == []
    salu = ["s_mov_b32 s4, 0", "buffer_load_dwordx4 v[18:21], v29, s[4:7], 0 offen nt"]
    assert vmem_sgpr_hazards(salu) == []
