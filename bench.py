"""Mimi encode+decode benchmark on one MI355X (prints one JSON line).

Workload: batch 1, 10 s of seeded synthetic 24 kHz
audio, 8 codebooks, FP32, the whole round trip replayed from a captured
hipGraph through ``MimiModel.forward``.  Inputs are resident in HBM before the
timed region.  ``value`` is audio-seconds per second; ``ms_per_step`` the mean
and ``median_ms`` the median round-trip latency.  The batch-16 configuration
(configs[2]: 10 s clips, last 4 zero-padded from 6 s) is reported beside it.

``parity`` compares each configuration's codes from the timed model with
the reference's (committed fixtures under ``tests/golden``) and reports the
float64 top-2 distance margins along the GPU's code chain.

``roofline`` describes the dominant kernel: its algorithmic FLOPs per launch
over its mean launch time, timed with HIP events on the stream it runs on.
``batch16.dominant_kernel`` times the same layer at the C3 shape, where its
grid runs many rounds of tiles (at C2 it is a single round).
``cpu_baseline`` times the repository's CPU oracle (the reference's portable
PyTorch path restated op for op) on the host cores, on the same 10 s input.

``roofline.traffic`` is the dominant kernel's HBM bytes per launch as read by
``rocprofv3 --pmc FETCH_SIZE`` and ``--pmc WRITE_SIZE`` on
``bench.py --dominant-only`` (which also runs a plain device copy of known
size to calibrate the counters); the figures live in
``profiles/dec_up4_convt_c2_hbm_traffic.md`` and are read from there.

The 100 s clip and the RVQ-heavy batch-64 / 32-codebook
configuration are reported as extra sections; the latter also
times the RVQ kernels alone (``rvq_only``: the split encode's distance
GEMMs against the FP32 MFMA peak, the decode gather-sum against HBM).
``c1`` is the 5 s clip on the GPU and ``cpu_baseline_c1`` the CPU oracle on
it (configs[0], the reference's CPU configuration).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --dominant-only [--iters N]   (counter runs)
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np
import torch

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "fast-mimi_amd"))

from fast_mimi_amd import MimiConfig, MimiModel, synthetic  # noqa: E402
from fast_mimi_amd import _native as nat  # noqa: E402
from fast_mimi_amd.diagnostics import code_margins  # noqa: E402
from fast_mimi_amd.flops import layer_table, roundtrip_flops  # noqa: E402

PEAK_FP32_TFLOPS = 157.3  # MI355X dense FP32 (matrix) peak
PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 (matrix) peak
PEAK_HBM_GBS = 8000.0
DOMINANT = "dec.up4"      # ConvTranspose1d 128->64, stride 4, 60000 -> 240000 rows


def time_steps(fn, steps: int, warmup: int) -> list[float]:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(steps):
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        stop.record()
        stop.synchronize()
        times.append(start.elapsed_time(stop))
    return times


def dominant_kernel(model: MimiModel, name: str, batch: int, samples: int, nq: int, iters: int):
    """Mean launch time of one contraction at its real shape, HIP events."""
    rt = model.runtime()
    row = next(r for r in layer_table(model.config, batch, samples, nq) if r[0] == name)
    flops = row[2]
    op = rt.layer_op(name, batch, samples)
    for _ in range(3):
        op()
    torch.cuda.synchronize()
    plan = nat.last_gemm_plan()  # the kernel the selection launched for this shape
    # The launches are captured in one hipGraph and replayed, so the events
    # bracket back-to-back kernels on the capture stream, not host launch gaps.
    graph = torch.cuda.CUDAGraph()
    # Captured in inference mode like the model's own graphs (they share the
    # default generator's graph state, created as an inference tensor).
    with torch.inference_mode(), torch.cuda.graph(graph):
        for _ in range(iters):
            op()
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    graph.replay()
    stop.record()
    stop.synchronize()
    ms = start.elapsed_time(stop) / iters
    del graph
    achieved = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "kernel": f"{plan} ({name}: {row[1]} rows={row[3]} K={row[4]} N={row[5]})",
            "flops_per_launch": flops, "avg_launch_ms": ms, "achieved": round(achieved, 3),
            "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4),
            "traffic": None,
            "note": ("FP32 contraction run as six bf16 MFMA products per operand pair (FP32-accurate); "
                     "achieved counts the algorithmic FP32 FLOPs against the FP32 MFMA peak"),
            "bf16_mfma_pipe_frac": round(6 * achieved / PEAK_BF16_TFLOPS, 4)}


def graph_ms(fn, iters: int) -> float:
    """Mean time of ``fn`` over ``iters`` back-to-back launches replayed from one
    hipGraph, by HIP events on the replay stream."""
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    graph.replay()
    stop.record()
    stop.synchronize()
    del graph
    return start.elapsed_time(stop) / iters


@torch.inference_mode()
def rvq_only(model: MimiModel, audio: torch.Tensor, nq: int, iters: int = 10) -> dict:
    """The RVQ kernels alone at their real shape (C5: 8000 frame vectors, 32
    codebooks): the split encode (distance GEMM + argmin + residual update per
    codebook, both chains) and the decode gather-sum, on the encoder's own
    projected RVQ inputs for this audio."""
    from fast_mimi_amd import ops

    rt = model.runtime()
    cfg = model.config
    h, B, T = rt.embeddings(audio)
    proj = rt.quantizer_inputs(h, B, T)
    M, vq, E = B * T, rt.vq, cfg.codebook_size
    n_sem = min(cfg.num_semantic_quantizers, nq)
    codes = torch.empty((B, nq, T), dtype=torch.int64, device=audio.device)
    wsb = nat.library().fm_rvq_split_workspace_bytes(M, vq, E)
    ws = torch.empty((wsb + 3) // 4, device=audio.device)
    q = torch.empty((M, 2 * vq), device=audio.device)

    def enc():
        ops.call("fm_rvq_encode_split", proj, 2 * vq, M, T, vq, E, n_sem, nq - n_sem,
                 rt.embeds, rt.embeds_t, rt.norms, codes, nq * T, ws, wsb)

    def dec():
        ops.call("fm_rvq_decode", codes, B, nq, T, cfg.num_semantic_quantizers, rt.embeds, E, vq, q)

    enc_ms = graph_ms(enc, iters)
    dec_ms = graph_ms(dec, iters)
    dist_flops = 2 * M * E * vq * nq            # distance GEMMs (cross terms x.e)
    gather_bytes = M * nq * (vq * 4 + 8) + M * 2 * vq * 4  # rows gathered + codes read + sums written
    enc_tf = dist_flops / (enc_ms * 1e-3) / 1e12
    dec_gbs = gather_bytes / (dec_ms * 1e-3) / 1e9
    return {"frames": M, "codebooks": nq, "entries": E, "dim": vq,
            "encode_ms": round(enc_ms, 4), "distance_gflop": round(dist_flops / 1e9, 2),
            # The reference's mm form contracts augmented rows (K = dim + 2).
            "distance_gflop_mm_form": round(2 * M * E * (vq + 2) * nq / 1e9, 2),
            "distance_tflops": round(enc_tf, 3), "distance_frac_fp32_mfma": round(enc_tf / PEAK_FP32_TFLOPS, 4),
            "decode_ms": round(dec_ms, 4), "gather_bytes": gather_bytes,
            "gather_gbs": round(dec_gbs, 1), "gather_frac_hbm": round(dec_gbs / PEAK_HBM_GBS, 4),
            "note": ("encode time covers every launch of fm_rvq_encode_split (per-codebook distance "
                     "MFMA + argmin + residual subtract, both chains); FLOPs count 2*M*E*D per codebook")}


TRAFFIC_FILE = REPO / "profiles" / "dec_up4_convt_c2_hbm_traffic.md"
COPY_BYTES = 256 << 20  # calibration copy: reads and writes this many bytes


def recorded_traffic() -> dict | None:
    """HBM bytes per launch of the dominant kernel from the committed counter summary.

    The file holds ``key: value`` lines; ``traffic_bytes_per_launch`` is the
    calibrated FETCH_SIZE + WRITE_SIZE per dispatch.
    """
    if not TRAFFIC_FILE.is_file():
        return None
    vals = {}
    for line in TRAFFIC_FILE.read_text().splitlines():
        if ":" in line and line.lstrip().startswith("- "):
            k, v = line.lstrip()[2:].split(":", 1)
            vals[k.strip().strip("`")] = v.strip().strip("`")
    try:
        return {"kernel": vals["kernel"], "bytes": float(vals["traffic_bytes_per_launch"]),
                "fetch": float(vals["fetch_bytes_per_launch"]),
                "write": float(vals["write_bytes_per_launch"])}
    except (KeyError, ValueError):
        return None


def dominant_only(iters: int) -> None:
    """Launches of the dominant contraction plus a calibration copy (for --pmc runs)."""
    dev = torch.device("cuda", 0)
    model = MimiModel(MimiConfig(), device=dev, seed=0)
    op = model.runtime().layer_op(DOMINANT, 1, 240_000)
    src = torch.randn(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(iters):
        op()
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"dominant": DOMINANT, "iters": iters, "copy_bytes": COPY_BYTES}), flush=True)


def cpu_baseline(audio: np.ndarray, mask: np.ndarray, nq: int, runs: int, what: str) -> dict:
    sys.path.insert(0, str(REPO))
    from oracle.mimi_oracle import MimiOracle
    from fast_mimi_amd.weights import seeded_state_dict

    # The GPU box grants this job 16 host cores whatever os.cpu_count() reports.
    cores = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(cores)
    cfg = MimiConfig()
    oracle = MimiOracle(cfg, {k: torch.from_numpy(v) for k, v in seeded_state_dict(cfg, 0).items()})
    a, m = torch.from_numpy(audio), torch.from_numpy(mask)
    times = []
    with torch.inference_mode():
        for _ in range(2):  # warm-up
            oracle.forward(a, m, nq)
        for _ in range(runs):
            t0 = time.perf_counter_ns()
            oracle.forward(a, m, nq)
            times.append((time.perf_counter_ns() - t0) / 1e6)
    med = statistics.median(times)
    total_s = sum(times) / 1e3
    seconds = audio.shape[0] * audio.shape[-1] / 24_000
    return {"value": round(seconds / (med / 1e3), 3), "unit": "audio-sec/sec", "cores": cores,
            "kind": "port", "median_ms": round(med, 2), "cpu": cpu_model(),
            "sample": f"{what}, nq={nq}, CPU oracle (PyTorch "
                      f"eager restatement of the reference model.py path), median of {runs} "
                      f"after 2 warm-ups ({total_s:.1f} s of timed CPU work), {cores} threads"}


GOLDEN = REPO / "tests" / "golden"


def reference_codes(name: str) -> dict[int, np.ndarray]:
    """The reference's codes for a configuration, per clip index (committed fixtures)."""
    if name == "c2":
        return {0: np.load(GOLDEN / "reference_golden.npz")["full_c2_codes"][0]}
    large = np.load(GOLDEN / "reference_golden_large.npz")
    if name == "c3":
        return dict(enumerate(large["c3_codes"]))
    if name == "c4":
        return {0: large["c4_codes"][0]}
    return {c: large[f"c5_clip{c}_codes"][0] for c in (0, 63)}


def parity(model, name: str, audio: torch.Tensor, codes: torch.Tensor) -> dict:
    """Codes of the timed run against the reference's, plus float64 near-tie margins."""
    got = codes.cpu().numpy()
    ref = reference_codes(name)
    differing = {c: int((got[c] != want.astype(np.int64)).sum()) for c, want in ref.items()}
    out = {"clips_checked": len(ref), "codes_differing_from_reference": sum(differing.values()),
           "codes_checked": int(sum(w.size for w in ref.values()))}
    out.update(code_margins(model, audio, codes))
    return out


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-runs", type=int, default=50)
    ap.add_argument("--no-extra", action="store_true", help="skip the 100 s and B64/nq32 sections")
    ap.add_argument("--dominant-only", action="store_true")
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-batch16", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(clips shard data-parallel across GPUs with no exchange; see DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    nat.library()
    if args.dominant_only:
        dominant_only(args.iters)
        return
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfg = MimiConfig()
    model = MimiModel(cfg, device=dev, seed=0)

    audio, mask, nq = synthetic.config_inputs("c2")
    a, m = torch.from_numpy(audio).to(dev), torch.from_numpy(mask).to(dev)
    times = time_steps(lambda: model(a, m, num_quantizers=nq), args.steps, args.warmup)
    checks = {"c2": parity(model, "c2", a, model(a, m, num_quantizers=nq).audio_codes)}
    mean_ms = statistics.fmean(times)
    med_ms = statistics.median(times)
    seconds = audio.shape[0] * audio.shape[-1] / 24_000
    flops = roundtrip_flops(cfg, 1, audio.shape[-1], nq)

    result = {
        "metric": "median ms, 10 s clip bs=1; audio-sec/sec at bs=16 (encode+decode, 8 codebooks)",
        "value": round(seconds / (med_ms / 1e3), 3),
        "unit": "audio-sec/sec (B=1, 10 s, median)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(mean_ms, 4), "median_ms": round(med_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded sinusoids + pink noise; seeded random-init weights)",
        "config": {"workload": "mimi encode+decode, B1 x 10 s @ 24 kHz, nq=8, hipGraph replay",
                   "global_batch": 1, "samples": int(audio.shape[-1]), "num_quantizers": nq},
        "pipeline_tflops": round(flops / (med_ms * 1e-3) / 1e12, 3),
        "pipeline_flops": flops,
    }
    a1, m1, nq1 = synthetic.config_inputs("c1")
    a1d, m1d = torch.from_numpy(a1).to(dev), torch.from_numpy(m1).to(dev)
    t1 = time_steps(lambda: model(a1d, m1d, num_quantizers=nq1), max(10, args.steps // 2), 3)
    result["c1"] = {"median_ms": round(statistics.median(t1), 4),
                    "audio_sec_per_sec": round(5.0 / (statistics.median(t1) / 1e3), 2)}
    # Same workload with the input in pageable host memory and codes + audio
    # copied back inside the timed region (PCIe-inclusive; not ``value``).
    a_host, m_host = torch.from_numpy(audio), torch.from_numpy(mask)

    def host_step():
        out = model(a_host.to(dev), m_host.to(dev), num_quantizers=nq)
        out.audio_codes.cpu()
        out.audio_values.cpu()

    th = time_steps(host_step, max(10, args.steps // 2), 3)
    result["host_io"] = {"median_ms": round(statistics.median(th), 4),
                         "audio_sec_per_sec": round(seconds / (statistics.median(th) / 1e3), 2),
                         "note": "input from pageable host memory, codes and audio copied back, "
                                 "all inside the timed region"}
    if not args.no_batch16:
        a16, m16, nq16 = synthetic.config_inputs("c3")
        a16d, m16d = torch.from_numpy(a16).to(dev), torch.from_numpy(m16).to(dev)
        t16 = time_steps(lambda: model(a16d, m16d, num_quantizers=nq16), max(5, args.steps // 5), 2)
        checks["c3"] = parity(model, "c3", a16d, model(a16d, m16d, num_quantizers=nq16).audio_codes)
        med16 = statistics.median(t16)
        f16 = roundtrip_flops(cfg, 16, a16.shape[-1], nq16)
        result["batch16"] = {"audio_sec_per_sec": round(16 * 10 / (med16 / 1e3), 2),
                             "median_ms": round(med16, 3),
                             "pipeline_tflops": round(f16 / (med16 * 1e-3) / 1e12, 3),
                             # The dominant kernel where its grid runs many rounds
                             # (at C2 it is one round of tiles).
                             "dominant_kernel": dominant_kernel(model, DOMINANT, 16, a16.shape[-1], nq16, 10)}
    if not args.no_extra:
        for key, cfg_name, steps in (("long100s", "c4", 10), ("rvq_b64_nq32", "c5", 5)):
            ax, mx, nqx = synthetic.config_inputs(cfg_name)
            axd, mxd = torch.from_numpy(ax).to(dev), torch.from_numpy(mx).to(dev)
            tx = time_steps(lambda: model(axd, mxd, num_quantizers=nqx), steps, 2)
            checks[cfg_name] = parity(model, cfg_name, axd, model(axd, mxd, num_quantizers=nqx).audio_codes)
            medx = statistics.median(tx)
            fx = roundtrip_flops(cfg, ax.shape[0], ax.shape[-1], nqx)
            result[key] = {"batch": int(ax.shape[0]), "samples": int(ax.shape[-1]),
                           "num_quantizers": nqx, "median_ms": round(medx, 3),
                           "audio_sec_per_sec": round(ax.shape[0] * ax.shape[-1] / 24_000 / (medx / 1e3), 2),
                           "pipeline_tflops": round(fx / (medx * 1e-3) / 1e12, 3)}
            if cfg_name == "c5":
                result[key]["rvq_only"] = rvq_only(model, axd, nqx)
            del axd, mxd
        model.release_graphs()
    result["parity"] = checks
    result["roofline"] = dominant_kernel(model, DOMINANT, 1, audio.shape[-1], nq, 50)
    tr = recorded_traffic()
    # The counter figures hold only for the kernel they were measured on.
    if tr is not None and result["roofline"]["kernel"].startswith(tr["kernel"] + " "):
        result["roofline"]["traffic"] = tr["bytes"]
        result["roofline"]["traffic_source"] = (f"{TRAFFIC_FILE.relative_to(REPO)} (rocprofv3 FETCH_SIZE + "
                                                "WRITE_SIZE of the same kernel and shape, not measured "
                                                "in this run)")
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(audio, mask, nq, args.cpu_runs,
                                              "B1 x 10 s (the bench workload itself)")
        result["speedup_vs_cpu"] = round(result["value"] / result["cpu_baseline"]["value"], 2)
        # C1 (B1 x 5 s), the configuration the reference's CPU path is quoted on.
        c1 = cpu_baseline(a1, m1, nq1, args.cpu_runs, "C1: B1 x 5 s")
        c1["gpu_median_ms"] = result["c1"]["median_ms"]
        c1["speedup_gpu_vs_cpu"] = round(c1["median_ms"] / result["c1"]["median_ms"], 2)
        result["cpu_baseline_c1"] = c1
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
