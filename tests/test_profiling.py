"""CPU tests of the rocprofv3 summary helpers (engine_amd/profiling.py) on
small synthetic trace and counter files in rocprofv3's CSV layout."""
import csv

from engine_amd import profiling as P

TRACE_FIELDS = ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp", "End_Timestamp"]


def _write_trace(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=TRACE_FIELDS)
        w.writeheader()
        for name, grid, t0, t1 in rows:
            w.writerow({"Kernel_Name": name, "Grid_Size_X": grid[0], "Grid_Size_Y": grid[1],
                        "Grid_Size_Z": grid[2], "Start_Timestamp": t0, "End_Timestamp": t1})


def test_short_name_demangles_and_drops_namespaces():
    assert P.short_name("_ZN8ribn_amd16gemv_wave_kernelILi12ELi1ELi1ELb1ELi2ELi8ELi1ELb0EEEvNS_11WaveGemvArgsE") == \
        "gemv_wave_kernel<12, 1, 1, true, 2, 8, 1, false>"
    assert P.short_name("void ribn_amd::(anonymous namespace)::attn_decode_kernel<4>(ribn_amd::AttnArgs)") == \
        "attn_decode_kernel<4>"


def test_trace_summary_groups_by_kernel_and_grid(tmp_path):
    f = tmp_path / "run_kernel_trace.csv"
    _write_trace(f, [("void ribn_amd::k<1>(int)", (64, 1, 1), 0, 2000),
                     ("void ribn_amd::k<1>(int)", (64, 1, 1), 3000, 7000),
                     ("void ribn_amd::k<1>(int)", (128, 1, 1), 8000, 9000)])
    rows = {(r[0], r[1]): r for r in P.trace_summary(str(tmp_path))}
    assert rows[("k<1>", 64)][2:] == (2, 3.0, 3.0, 2.0)
    assert rows[("k<1>", 128)][2] == 1


def test_decode_steps_windows_by_argmax_grid(tmp_path):
    # batch 1 (argmax grid 1024): three steps of gemv (2 us) + argmax (1 us);
    # batch 8 (grid 8192) afterwards: two steps of gemv (5 us) + argmax (1 us),
    # with 4x2x1 grids to check X*Y*Z.
    rows, t = [], 0
    for _ in range(3):
        rows.append(("void ribn_amd::gemv<1>(int)", (4096, 1, 1), t, t + 2000))
        rows.append(("void ribn_amd::(anonymous namespace)::argmax_kernel(int)", (1024, 1, 1), t + 2000, t + 3000))
        t += 3000
    for _ in range(2):
        rows.append(("void ribn_amd::gemv<8>(int)", (4, 2, 1), t, t + 5000))
        rows.append(("void ribn_amd::(anonymous namespace)::argmax_kernel(int)", (1024, 8, 1), t + 5000, t + 6000))
        t += 6000
    _write_trace(tmp_path / "x_kernel_trace.csv", rows)
    w = {r["argmax_grid"]: r for r in P.decode_steps_summary(str(tmp_path), steps=1)}
    assert sorted(w) == [1024, 8192]
    b1 = w[1024]
    assert b1["dispatches"] == 2 and b1["span_us"] == 3.0 and b1["busy_us"] == 3.0
    assert b1["kernels"][0] == ("gemv<1>", 4096, 1.0, 2.0, 2.0)
    b8 = w[8192]
    assert b8["kernels"][0] == ("gemv<8>", 8, 1.0, 5.0, 5.0)
    # more steps than the trace holds: that batch size is left out
    assert [r["argmax_grid"] for r in P.decode_steps_summary(str(tmp_path), steps=2)] == [1024]


def test_decode_steps_end_at_the_final_selection_launch(tmp_path):
    # the two-launch greedy selection: slices (not a step boundary), then the
    # final merge (64 threads per member) ends the step
    rows, t = [], 0
    for _ in range(2):
        rows.append(("void ribn_amd::gemv<1>(int)", (4096, 1, 1), t, t + 2000))
        rows.append(("ribn_amd::(anonymous namespace)::argmax_slice_kernel(float const*, int, int, uint2*)",
                     (16384, 1, 1), t + 2000, t + 2500))
        rows.append(("ribn_amd::(anonymous namespace)::argmax_final_kernel(uint2 const*, int)", (64, 1, 1),
                     t + 2500, t + 3000))
        t += 3000
    _write_trace(tmp_path / "x_kernel_trace.csv", rows)
    (w,) = P.decode_steps_summary(str(tmp_path), steps=1)
    assert w["argmax_grid"] == 64 and w["dispatches"] == 3 and w["busy_us"] == 3.0


def test_resource_remarks_parse():
    """The build's resource report reads the compiler's kernel-resource-usage
    remarks (engine_amd/build.py --resource-report)."""
    from engine_amd import build as B
    tag = " [-Rpass-analysis=kernel-resource-usage]"
    text = "\n".join([
        "engine_amd/csrc/q8_1.hip:39:1: remark: Function Name: _ZN8ribn_amd4kernEv" + tag,
        "   39 |   uint32_t blocks) {",
        "engine_amd/csrc/q8_1.hip:39:1: remark:     TotalSGPRs: 16" + tag,
        "engine_amd/csrc/q8_1.hip:39:1: remark:     VGPRs: 14" + tag,
        "engine_amd/csrc/q8_1.hip:39:1: remark:     AGPRs: 0" + tag,
        "engine_amd/csrc/q8_1.hip:39:1: remark:     ScratchSize [bytes/lane]: 8" + tag,
        "engine_amd/csrc/q8_1.hip:39:1: remark:     Occupancy [waves/SIMD]: 8" + tag,
        "engine_amd/csrc/q8_1.hip:39:1: remark:     SGPRs Spill: 0" + tag,
        "engine_amd/csrc/q8_1.hip:39:1: remark:     VGPRs Spill: 2" + tag,
        "engine_amd/csrc/q8_1.hip:39:1: remark:     LDS Size [bytes/block]: 4096" + tag,
        "engine_amd/csrc/q8_1.hip:90:1: remark: Function Name: _ZN8ribn_amd5otherEv" + tag,
        "engine_amd/csrc/q8_1.hip:90:1: remark:     VGPRs: 40" + tag,
    ])
    k = B.parse_resource_remarks(text)
    assert k[0] == {"source": "q8_1.hip", "kernel": "_ZN8ribn_amd4kernEv", "sgpr": 16, "vgpr": 14, "agpr": 0,
                    "scratch": 8, "occupancy": 8, "sgpr_spill": 0, "vgpr_spill": 2, "lds": 4096}
    assert k[1] == {"source": "q8_1.hip", "kernel": "_ZN8ribn_amd5otherEv", "vgpr": 40}
    assert B._short_name("void ribn_amd::(anonymous namespace)::k<1, (x)2>(ribn_amd::A)") == "k<1, (x)2>"
    # _Float16 parameters (DF16_) that binutils' c++filt leaves mangled still read as names
    assert B._demangle(["_ZN8ribn_amd12qgemm_kernelILi12ELi4ELi8EEEvPKhjPKDF16_PKfPfS7_iiii",
                        "_ZN8ribn_amd14act_f16_kernelILb0ELb1ELi1EEEvPKvPKffiPDF16_PfS4_"]) == [
        "qgemm_kernel<12, 4, 8>", "act_f16_kernel<false, true, 1>"]


def test_prompt_summary_keeps_prompt_kernels_only(tmp_path):
    # two prompts of (act 1 us, qgemm 10 us, attention 4 us), with decode
    # kernels around them that the summary leaves out
    rows, t = [], 0
    for _ in range(2):
        for name, dur in (("void ribn_amd::act_f16_kernel<false, true, 0>(void const*)", 1000),
                          ("void ribn_amd::qgemm_tile_kernel<12, 3, 8>(int)", 10000),
                          ("void ribn_amd::(anonymous namespace)::attn_prefill_kernel<4>(ribn_amd::PrefillAttnArgs)",
                           4000),
                          ("void ribn_amd::gemv_f32_kernel<12>(int)", 3000)):
            rows.append((name, (256, 1, 1), t, t + dur))
            t += dur + 100
    f = tmp_path / "run_kernel_trace.csv"
    _write_trace(f, rows)
    w = P.prompt_summary(str(tmp_path), prompts=2)
    names = [k[0] for k in w["kernels"]]
    assert names == ["qgemm_tile_kernel<12, 3, 8>", "attn_prefill_kernel<4>", "act_f16_kernel<false, true, 0>"]
    assert w["kernels"][0][2:] == (1.0, 10.0, 10.0)
    assert abs(w["busy_us"] - 15.0) < 1e-9
