"""bench.py's readers of the committed profiles (CPU only): the HBM traffic per launch
and the measured ceilings that its JSON line carries beside the published peaks."""
import bench


def test_measured_ceilings_parse():
    """Every workload with a measured ceiling reads it from its profile, in its unit,
    below the published peak, with frac = achieved / ceiling."""
    for wl, unit, peak in (("decode_sweep_llama2_7b", "GB/s", bench.HBM_PEAK_GBS),
                           ("decode_sweep_llama2_70b", "GB/s", bench.HBM_PEAK_GBS),
                           ("prefill_sweep_llama2_70b", "TFLOP/s", bench.SPARSE_F16_PEAK_TFLOPS)):
        c = bench.ceiling_from_profile(wl, 1000.0)
        assert c is not None, wl
        assert c["unit"] == unit and 0 < c["value"] < peak, (wl, c)
        assert c["frac"] == round(1000.0 / c["value"], 4)
        assert c["source"].startswith("profiles/")
    assert bench.ceiling_from_profile("w3_values_llama2_7b", 1.0) is None


def test_traffic_parses():
    """The decode sweeps' traffic per launch is within 1.0-1.3x their algorithmic
    weight bytes per launch (25/64 K N averaged over the 20 calls)."""
    for wl, shapes in (("decode_sweep_llama2_7b", bench.LLAMA7B), ("decode_sweep_llama2_70b", bench.LLAMA70B)):
        t = bench.traffic_from_profile(wl)
        alg = sum(25 * K * N // 64 for _, K, N in shapes) / len(shapes)
        assert t is not None and 1.0 <= t / alg <= 1.3, (wl, t, alg)
