"""The build-time check of the GEMM's inline-asm LDS reads (brimkern_amd/check_lds_reads.py) on
hand-written disassembly: a register of an LDS read touched before `s_waitcnt lgkmcnt(0)` is reported,
the same code with the wait first is not, and kernels outside the checked set are skipped."""
from brimkern_amd.check_lds_reads import check

HEAD = "0000000000001000 <{}>:\n"


def body(lines):
    return "".join(f"\t{l}  // 0000000010{i:02X}: 00000000\n" for i, l in enumerate(lines))


def test_touch_before_wait_is_reported():
    text = HEAD.format("brik_gemm_q4_96x1w8") + body([
        "ds_read_b128 v[2:5], v44 offset:64",
        "v_lshlrev_b32_e32 v2, 2, v18",          # reuses v2 while the read may still write it
        "s_waitcnt lgkmcnt(0)",
    ])
    bad = check(text)
    assert len(bad) == 1 and "v[2]" in bad[0]


def test_use_after_wait_is_clean():
    text = HEAD.format("brik_gemmg_q4_64x1w8") + body([
        "ds_read_b128 v[2:5], v44",
        "ds_read_u16 v9, v40 offset:2",
        "v_and_or_b32 v10, v11, v12, v13",       # unrelated registers
        "s_waitcnt lgkmcnt(0)",
        "v_mfma_f32_32x32x16_f16 a[0:15], v[2:5], v[14:17], a[0:15]",
        "v_mov_b32_e32 v9, 0",
    ])
    assert check(text) == []


def test_window_spans_branches_and_other_kernels_are_skipped():
    text = HEAD.format("brik_gemm_q8_64x1") + body([
        "ds_read_b128 v[6:9], v1",
        "s_cbranch_scc1 65530",
        "v_add_u32_e32 v7, s0, v3",               # after the branch, before any wait
    ]) + HEAD.format("brik_gemm_sk_q4_k4") + body([
        "ds_read_b128 v[6:9], v1",
        "v_add_u32_e32 v7, s0, v3",               # compiler-tracked reads: not checked
    ])
    bad = check(text)
    assert len(bad) == 1 and bad[0].startswith("brik_gemm_q8_64x1")


def at(lines, base=0x1000):
    """Instructions 4 bytes apart (branch offsets count 4-byte words from the next instruction)."""
    return "".join(f"\t{l}  // {base + 4 * i:012X}: 00000000\n" for i, l in enumerate(lines))


def test_loop_back_edge_is_followed():
    """A read at the bottom of a loop whose register is used at the loop head, reached only by the back
    edge (address order alone never sees the use after the read)."""
    text = HEAD.format("brik_gemm_q4_64x1") + at([
        "v_add_u32_e32 v20, v7, v3",              # 0x1000: loop head, uses v7
        "ds_read_b128 v[6:9], v1",                # 0x1004
        "s_cbranch_scc1 65533",                   # 0x1008: -3 words -> 0x1000
        "s_waitcnt lgkmcnt(0)",                   # 0x100c
        "s_endpgm",
    ])
    bad = check(text)
    assert len(bad) == 1 and "v[7]" in bad[0] and "v_add_u32" in bad[0]


def test_wait_on_every_path_is_clean():
    text = HEAD.format("brik_gemm_q4_64x1") + at([
        "s_waitcnt lgkmcnt(0)",                   # 0x1000: loop head waits first
        "v_add_u32_e32 v20, v7, v3",
        "ds_read_b128 v[6:9], v1",
        "s_cbranch_scc1 65532",                   # 0x100c: -4 words -> 0x1000
        "s_waitcnt lgkmcnt(0)",
        "v_mov_b32_e32 v7, 0",
        "s_endpgm",
    ])
    assert check(text) == []


def test_unconditional_branch_skips_fallthrough():
    text = HEAD.format("brik_gemm_q4_64x1") + at([
        "ds_read_b128 v[6:9], v1",                # 0x1000
        "s_branch 1",                             # 0x1004: +1 word -> 0x100c
        "v_mov_b32_e32 v7, 0",                    # 0x1008: never reached
        "s_waitcnt lgkmcnt(0)",                   # 0x100c
        "v_mov_b32_e32 v7, 0",
        "s_endpgm",
    ])
    assert check(text) == []


def test_counted_wait_retires_older_reads_only():
    """LDS reads complete in order: lgkmcnt(1) retires every read but the last one issued."""
    text = HEAD.format("brik_gemm_q4_128x1w8") + body([
        "ds_read_b128 v[66:69], v0",
        "ds_read_b128 v[50:53], v1",
        "s_waitcnt lgkmcnt(1)",
        "v_mad_i64_i32 v[66:67], s[2:3], v0, s10, 0",   # the older read has landed
        "v_mul_f32_e32 v1, v54, v50",                   # the newer one may not have
        "s_waitcnt lgkmcnt(0)",
    ])
    bad = check(text)
    assert len(bad) == 1 and "v[50]" in bad[0] and "v_mul_f32" in bad[0]


def test_counted_wait_with_a_scalar_load_in_flight_retires_nothing():
    """A scalar load may complete before an earlier LDS read, so lgkmcnt(1) then guarantees nothing."""
    text = HEAD.format("brik_gemm_q4_128x1w8") + body([
        "ds_read_b128 v[66:69], v0",
        "s_load_dwordx2 s[4:5], s[0:1], 0x0",
        "s_waitcnt lgkmcnt(1)",
        "v_mov_b32_e32 v66, 0",
        "s_waitcnt lgkmcnt(0)",
    ])
    bad = check(text)
    assert len(bad) == 1 and "v[66]" in bad[0]


def test_join_keeps_the_younger_age():
    """Paths that meet with the same read at different ages: the wait after the join must cover the
    path on which fewer operations followed it."""
    text = HEAD.format("brik_gemm_q4_64x1") + at([
        "ds_read_b128 v[6:9], v1",                # 0x1000
        "s_cbranch_scc1 1",                       # 0x1004: -> 0x100c, the read still at age 0
        "ds_read_b128 v[10:13], v1",              # 0x1008: the read at age 1 on this path
        "s_waitcnt lgkmcnt(1)",                   # 0x100c
        "v_mov_b32_e32 v7, 0",                    # not retired on the branch path
        "s_waitcnt lgkmcnt(0)",
        "s_endpgm",
    ])
    bad = check(text)
    assert len(bad) == 1 and "v[7]" in bad[0]
