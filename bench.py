"""Benchmark of the quantized-weight hot path on one MI355X.

Headline (the JSON line's value): Q4_K dequantisation of a 14B-DiT FFN weight pair, 13824 x 5120 and
5120 x 13824, float32 N(0, 0.02) weights (seed 1234 / 1235) encoded to Q4_K, dequantised with MID float16 to
bfloat16 output. One step = both matrices (two launches of the same kernel). Inputs are resident in HBM before
the timed region; each step works on the next of four copies of inputs and outputs (1.45 GB in all), so the
256 MB last-level cache cannot serve one step's bytes to the next.

Other rows of the workload list are reported under "also": Q8_0 dequantisation of a 5120 x 5120 weight.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import importlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = "comfyui-weightferry_amd"
HBM_PEAK_GBS = 8000.0
ROTATE = 4


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true", help="leave out the CPU baseline leg")
    return ap.parse_args()


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def dequant_leg(torch, native, raws, shapes, qtype, mid, out_dt, steps, warmup):
    """Time `steps` steps of dequantising every matrix once, launched back to back on torch's current stream with
    events at both ends of the timed region on that stream. Returns (ms per step, mean ms per launch, bytes/step);
    the launches are all of one kernel, so the mean per launch is that kernel's average duration."""
    lib = native.lib()
    dev = torch.device("cuda:0")
    stream = native.stream_of(dev)
    out_torch = {0: torch.float16, 1: torch.bfloat16, 2: torch.float32}[out_dt]
    ins = [[torch.from_numpy(r).to(dev) for r in raws] for _ in range(ROTATE)]
    outs = [[torch.empty(s, dtype=out_torch, device=dev) for s in shapes] for _ in range(ROTATE)]
    nvals = [s[0] * s[1] for s in shapes]
    algo = sum(r.size for r in raws) + sum(n * outs[0][0].element_size() for n in nvals)

    def launch(r, m):
        rc = lib.wf_dequant(ins[r][m].data_ptr(), ins[r][m].numel(), qtype, mid, out_dt, outs[r][m].data_ptr(),
                            nvals[m], stream)
        if rc != 0:
            raise RuntimeError(native.last_error())

    for i in range(warmup):
        for m in range(len(shapes)):
            launch(i % ROTATE, m)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        for m in range(len(shapes)):
            launch(i % ROTATE, m)
    t1.record()
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / steps
    del ins, outs
    torch.cuda.empty_cache()
    return ms_step, ms_step / len(shapes), algo


def cpu_baseline_dequant(torch, raw, qtype, rows, cols, budget_s=12.0):
    """The reference's CPU path (ComfyUI-GGUF's torch op chain, restated in oracle.torch_chain) on the first
    `rows` rows of one weight; GB/s with the same byte accounting as the GPU leg."""
    from oracle import torch_chain
    ts = torch_chain.TYPE_SIZE[qtype]
    per = torch_chain.BLOCK_SIZE[qtype]
    nbytes = rows * cols // per * ts
    sample = torch.from_numpy(raw[:nbytes].copy())
    cores = min(16, os.cpu_count() or 1)
    torch.set_num_threads(cores)
    for _ in range(2):
        torch_chain.dequantize(sample, qtype, (rows, cols), torch.float16, torch.bfloat16)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 10 and time.perf_counter() < t_end:
        t = time.perf_counter()
        torch_chain.dequantize(sample, qtype, (rows, cols), torch.float16, torch.bfloat16)
        times.append(time.perf_counter() - t)
    times.sort()
    med = times[len(times) // 2]
    algo = nbytes + rows * cols * 2
    return {"value": round(algo / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"ComfyUI-GGUF torch op chain (oracle/torch_chain.py) on CPU, Q4_K -> bf16 (MID f16), "
                      f"first {rows} rows of the 13824x5120 weight, median of {len(times)} runs"}


def main():
    args = _args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the one-GPU throughput is the reported value)", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, ROOT)
    import numpy as np  # noqa: F401
    import torch

    from oracle import encode

    native = importlib.import_module(PKG + "._native")
    native.lib()
    _log(f"library {native.LIB_PATH}")

    shapes = [(13824, 5120), (5120, 13824)]
    t = time.perf_counter()
    raws = [encode.encode_q4_k(encode.weights(s, seed=1234 + i)) for i, s in enumerate(shapes)]
    _log(f"encoded Q4_K pair in {time.perf_counter() - t:.1f} s")

    ms_step, kern_ms, algo = dequant_leg(torch, native, raws, shapes, 12, 0, 1, args.steps, args.warmup)
    value = algo / (ms_step / 1e3) / 1e9
    per_launch = algo / len(shapes)
    achieved = per_launch / (kern_ms / 1e3) / 1e9
    _log(f"Q4_K pair: {ms_step * 1e3:.1f} us/step, kernel {kern_ms * 1e3:.1f} us, {value:.0f} GB/s")

    also = {}
    # MID float32 on the same pair
    ms32, k32, _ = dequant_leg(torch, native, raws, shapes, 12, 2, 1, max(5, args.steps // 2), 3)
    also["q4_k_pair_mid_f32"] = {"GB/s": round(algo / (ms32 / 1e3) / 1e9, 1),
                                 "kernel_us": round(k32 * 1e3, 2)}
    # Q8_0 5120 x 5120 (MID float16 and float32 -> bf16)
    q8 = [encode.encode_q8_0(encode.weights((5120, 5120), seed=1234))]
    for mid, name in ((0, "q8_0_5120sq_mid_f16"), (2, "q8_0_5120sq_mid_f32")):
        ms8, k8, a8 = dequant_leg(torch, native, q8, [(5120, 5120)], 8, mid, 1, args.steps, args.warmup)
        also[name] = {"GB/s": round(a8 / (k8 / 1e3) / 1e9, 1), "kernel_us": round(k8 * 1e3, 2),
                      "frac": round(a8 / (k8 / 1e3) / 1e9 / HBM_PEAK_GBS, 3), "bytes": a8}
    cpu = None
    if not args.skip_cpu:
        cpu = cpu_baseline_dequant(torch, raws[0], 12, 512, 5120)
        _log(f"cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads")

    line = {
        "metric": "dequant HBM GB/s (% peak); int8/bf16 GEMM TFLOPS; streamed-block ms/step",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: fp32 N(0,0.02) weights, seed 1234/1235, encoded to Q4_K",
        "config": {"workload": "Q4_K dequant of a 14B-DiT FFN pair 13824x5120 + 5120x13824 -> bf16 (MID f16)",
                   "bytes_per_step": algo, "rotating_copies": ROTATE},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "wf::deq_items<wf::Q45_K<12, f16, bf16>>", "kernel_us": round(kern_ms * 1e3, 2),
                     "bytes_per_launch": per_launch},
        "cpu_baseline": cpu,
        "also": also,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
