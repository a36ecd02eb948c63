"""Benchmark of the quantized-weight hot path on one MI355X.

Headline (the JSON line's value): Q4_K dequantisation of a 14B-DiT FFN weight pair, 13824 x 5120 and
5120 x 13824, float32 N(0, 0.02) weights (seed 1234 / 1235) encoded to Q4_K, dequantised with MID float16 to
bfloat16 output. One step = both matrices (two launches of the same kernel). Inputs are resident in HBM before
the timed region; each step works on the next of four copies of inputs and outputs (1.45 GB in all), so the
256 MB last-level cache cannot serve one step's bytes to the next.

Other rows of the workload list are reported under "also":
  * Q8_0 dequantisation of a 5120 x 5120 weight (MID float16 and float32) and of the FFN pair;
  * what HBM delivers, with the same rotation, to a kernel that only moves the bytes of a dequantisation launch
    (the Q4_K 13824 x 5120 launch, Q8_0 / Q4_0 / Q6_K 5120 x 5120) in the nearest read:write mix (1:2 or 2:7), and
    the Q4_K / Q8_0 launches as a fraction of it;
  * every other GGML format at 5120 x 5120 -> bf16 (MID float16): Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q5_K / Q6_K encoded
    from the same N(0, 0.02) weights, Q2_K / Q3_K as random blocks with typical float16 scales;
  * the int8 W8A8 linear at M in {1024, 4096, 16384}, K = 5120, N in {5120, 13824} (per-token int8 activations,
    per-channel int8 weights, int32 accumulation, bf16 out), and the row quantiser;
  * fused Q5_K / Q6_K dequant + bf16 GEMM over the linears of one Wan-2.1-14B block at 4096 tokens, next to the
    two-step flow (wf_dequant, then torch's bf16 GEMM), and the same linears at 32 tokens (Q4_K / Q5_K / Q6_K, the
    fused kernel's few-rows form);
  * the LoRA add on a Q4_K 13824 x 5120 weight: the first LoRA fused into the dequantisation and a later LoRA
    onto the bf16 weight (float32 difference of n values each);
  * 40 streamed Wan-14B blocks of Q4_K from pinned host memory through 2 GPU slots, 4096 tokens (ms/step, H2D
    GB/s, share of the copy time hidden behind compute);
  * chunk (sub-block) streaming of the same 40 blocks: 96 MB chunks of a block's linears through 4 GPU slots;
  * the SSD tier: the same 40 blocks as a GGUF file on local disk, the reader ring's O_DIRECT read rate, and the
    streamed forward with half the blocks read from the file on every step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--only-headline] [--legs LEGS]
--legs (comma list of headline, ceiling, formats, lora, int8, fused, streaming, chunk, ssd; default all) runs only
those legs, for profiling one kernel family; without the headline leg the printed line holds the legs' figures only.
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
ROTATE_BYTES = 1_200_000_000


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true", help="leave out the CPU baseline leg")
    ap.add_argument("--only-headline", action="store_true", help="the Q4_K dequant leg only")
    ap.add_argument("--legs", default="all",
                    help="comma list: headline, ceiling, formats, lora, int8, fused, streaming, chunk, ssd")
    a = ap.parse_args()
    a.legs = {"headline"} if a.only_headline else (
        {"headline", "ceiling", "formats", "lora", "int8", "fused", "streaming", "chunk", "ssd"} if a.legs == "all"
        else set(a.legs.split(",")))
    return a


WARM_S = 0.05


def _warm_clock(torch, fn, seconds=WARM_S):
    """Call fn() until `seconds` have passed (at least once). MI355X raises its clock over tens of milliseconds of
    load after an idle spell (host-side set-up between measurements): the first ~10 calls of a 0.5 ms kernel ran
    10 % slower than later ones, so whichever variant was timed first looked slower."""
    t0 = time.perf_counter()
    while True:
        fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return


def _timed(torch, fn, n, warm):
    """Mean ms of fn() over n back-to-back calls on torch's current stream (events at both ends), after `warm`
    calls and at least WARM_S seconds of calls."""
    _warm_clock(torch, fn)
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(n):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / n


def int8_leg(torch, native):
    """W8A8 linear rows: TOPS of wf_linear_i8 and GB/s of wf_quant_rows_i8 (plain per-token)."""
    lib = native.lib()
    dev = torch.device("cuda:0")
    st = native.stream_of(dev)
    K = 5120
    out = {}
    g = torch.Generator(device=dev).manual_seed(1234)
    for M in (1024, 4096, 16384):
        x = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
        xq = torch.empty((M, K), dtype=torch.int8, device=dev)
        xs = torch.empty(M, dtype=torch.float32, device=dev)
        msq = _timed(torch, lambda: lib.wf_quant_rows_i8(x.data_ptr(), M, K, 0, xq.data_ptr(), xs.data_ptr(), st),
                     20, 3)
        out[f"quant_rows_plain_M{M}"] = {"us": round(msq * 1e3, 2),
                                         "GB/s": round((3 * M * K + 4 * M) / msq / 1e6, 1)}
        for N in (5120, 13824):
            w = torch.randn((N, K), device=dev, generator=g) * 0.02
            ws = (w.abs().amax(dim=1) / 127).float()
            wq = torch.clamp(torch.round(w / ws[:, None]), -127, 127).to(torch.int8)
            del w
            y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            ms = _timed(torch, lambda: lib.wf_linear_i8(xq.data_ptr(), wq.data_ptr(), xs.data_ptr(), ws.data_ptr(),
                                                        None, y.data_ptr(), 1, M, N, K, st), 10, 2)
            tops = 2 * M * N * K / ms / 1e9
            out[f"gemm_M{M}_N{N}"] = {"us": round(ms * 1e3, 1), "TOPS": round(tops, 1),
                                      "frac_of_5000": round(tops / 5000, 3)}
            del wq, y
        del x, xq
    # the same 16384 x 5120 x 5120 product on all-ones operands (the fewest toggling bits: the chip keeps a higher
    # clock under its power budget) and hipBLASLt's int8 GEMM (torch._int_mm, int32 out, no epilogue) on random
    # operands: the first is the kernel's rate without the power cap's clock reduction, the second the library's
    # rate under the same cap
    M, N = 16384, 5120
    xq = torch.ones((M, K), dtype=torch.int8, device=dev)
    wq = torch.ones((N, K), dtype=torch.int8, device=dev)
    xs = torch.ones(M, dtype=torch.float32, device=dev)
    ws = torch.full((N,), 1.0 / K, dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ms = _timed(torch, lambda: lib.wf_linear_i8(xq.data_ptr(), wq.data_ptr(), xs.data_ptr(), ws.data_ptr(), None,
                                                y.data_ptr(), 1, M, N, K, st), 10, 2)
    out["gemm_M16384_N5120_ones"] = {"us": round(ms * 1e3, 1), "TOPS": round(2 * M * N * K / ms / 1e9, 1)}
    xq = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
    wq = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
    wt = wq.t()
    ms = _timed(torch, lambda: torch._int_mm(xq, wt), 10, 2)
    out["hipblaslt_int_mm_M16384_N5120"] = {"us": round(ms * 1e3, 1), "TOPS": round(2 * M * N * K / ms / 1e9, 1)}
    del xq, wq, wt, xs, ws, y
    torch.cuda.empty_cache()
    return out


WAN_LINEARS = [("q", 5120, 5120), ("k", 5120, 5120), ("v", 5120, 5120), ("o", 5120, 5120),
               ("ffn_up", 13824, 5120), ("ffn_down", 5120, 13824)]


def fused_leg(torch, native):
    """One Wan-14B block's linears at 4096 tokens with Q5_K / Q6_K weights: the fused kernel and the two-step
    flow (wf_dequant to bf16, then a bf16 GEMM: torch's, hipBLASLt, and the library's wf_linear_bf16, which the
    GGUF linear's two-step flow takes at this row count)."""
    sys.path.insert(0, ROOT)
    encode = importlib.import_module(PKG + ".gguf_encode")
    lib = native.lib()
    dev = torch.device("cuda:0")
    st = native.stream_of(dev)
    M = 4096
    res = {}
    for qt, name in ((13, "q5_k"), (14, "q6_k")):
        tf = tu = th = 0.0
        flops = wbytes = 0
        for lname, N, K in WAN_LINEARS:
            raw = torch.from_numpy(encode.encode(encode.weights((N, K), seed=N + K), qt)).to(dev)
            x = torch.randn((M, K), device=dev).to(torch.bfloat16)
            y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            w = torch.empty((N, K), dtype=torch.bfloat16, device=dev)

            def fused():
                lib.wf_linear_gguf(x.data_ptr(), M, K, raw.data_ptr(), raw.numel(), qt, N, None, y.data_ptr(), 0, st)

            def two_step():
                lib.wf_dequant(raw.data_ptr(), raw.numel(), qt, 0, 1, w.data_ptr(), N * K, st)
                torch.matmul(x, w.t(), out=y)

            def two_step_hand():
                lib.wf_dequant(raw.data_ptr(), raw.numel(), qt, 0, 1, w.data_ptr(), N * K, st)
                lib.wf_linear_bf16(x.data_ptr(), w.data_ptr(), None, y.data_ptr(), M, N, K, st)
            tf += _timed(torch, fused, 10, 2)
            tu += _timed(torch, two_step, 10, 2)
            th += _timed(torch, two_step_hand, 10, 2)
            flops += 2 * M * N * K
            wbytes += raw.numel()
            del raw, x, y, w
        res[name] = {"fused_ms": round(tf, 3), "fused_TFLOPS": round(flops / tf / 1e9, 1),
                     "fused_frac_of_2500": round(flops / tf / 1e9 / 2500, 3),
                     "two_step_ms": round(tu, 3), "two_step_TFLOPS": round(flops / tu / 1e9, 1),
                     "two_step_hand_ms": round(th, 3), "two_step_hand_TFLOPS": round(flops / th / 1e9, 1),
                     "flop": flops, "weight_bytes": wbytes}
    # few activation rows (128 and 32 tokens, and one token): the fused kernel's few-rows form streams each weight
    # once, its panel form once per 16 MT rows. "cold": every call reads another copy of the weight, the copies of a
    # layer spanning > 600 MB, so MI355X's 256 MB last-level cache cannot serve a call from the one before (a weight
    # in a real forward was last read a step earlier); "warm": the same weight every call. Every row count goes
    # through fused_gguf.fused_linear, the drop-in's choice of form with its workspace: the panel form in K slices at
    # 128 rows (Q8_0 in 64-row panels), and at 32 rows for the K-quants' deep ffn_down (K >= 2 N); the whole-rows form
    # at one token (Q4_K / Q5_K for the 5120-wide outputs, Q6_K and Q8_0 for all six); the few-rows form otherwise.
    fg = importlib.import_module(PKG + ".enhancers.fused_gguf")
    for rows in (128, 32, 1):
        for qt, name in ((12, "q4_k"), (13, "q5_k"), (14, "q6_k"), (8, "q8_0")):
            tf = tc = tu = 0.0
            wbytes = 0
            for lname, N, K in WAN_LINEARS:
                raw = torch.from_numpy(encode.encode(encode.weights((N, K), seed=N + K), qt)).to(dev)
                ncopy = max(2, -(-600_000_000 // raw.numel()))
                copies = [raw] + [raw.clone() for _ in range(ncopy - 1)]
                x = torch.randn((rows, K), device=dev).to(torch.bfloat16)
                y = torch.empty((rows, N), dtype=torch.bfloat16, device=dev)
                w = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
                turn = [0]

                def fused(r=raw):
                    fg.fused_linear(x, r, qt, (N, K))

                def fused_cold():
                    turn[0] += 1
                    fused(copies[turn[0] % ncopy])

                def two_step():
                    lib.wf_dequant(raw.data_ptr(), raw.numel(), qt, 0, 1, w.data_ptr(), N * K, st)
                    torch.matmul(x, w.t(), out=y)
                tf += _timed(torch, fused, 20, 3)
                tc += _timed(torch, fused_cold, 2 * ncopy, ncopy)
                tu += _timed(torch, two_step, 20, 3)
                wbytes += raw.numel()
                del raw, copies, x, y, w
            torch.cuda.empty_cache()
            res[f"{name}_{rows}_token{'s' if rows > 1 else ''}"] = {
                "fused_us_cold": round(tc * 1e3, 1), "fused_us_warm": round(tf * 1e3, 1),
                "two_step_us": round(tu * 1e3, 1), "fused_weight_GBps_cold": round(wbytes / (tc / 1e3) / 1e9, 1),
                "fused_weight_GBps_warm": round(wbytes / (tf / 1e3) / 1e9, 1), "weight_bytes": wbytes}
    torch.cuda.empty_cache()
    return res


def _resident_check(torch, sm, model, x, ctx, y_stream, dev):
    """The reference's criterion for streaming (tests/test_streaming.py:222, torch.equal): tear the streaming down
    with the blocks' weights moved onto the GPU, run the same forward resident and compare it with the last streamed
    output bit for bit."""
    sm.teardown(device=dev)
    with torch.no_grad():
        y_res = model(x, ctx)
    torch.cuda.synchronize()
    return bool(torch.equal(y_res.view(torch.int16), y_stream.view(torch.int16)))


def streaming_leg(torch, native, n_blocks=40, steps=10):
    """40 Wan-14B blocks with Q4_K weights streamed from pinned host memory through 2 GPU slots (4096 tokens)."""
    syn = importlib.import_module(PKG + ".streaming.synthetic")
    dn = importlib.import_module(PKG + ".streaming.dit_node")
    prof_mod = importlib.import_module(PKG + ".streaming.profiler")
    dev = torch.device("cuda:0")
    t = time.perf_counter()
    model = syn.WanLikeStack(n_blocks=n_blocks, qtype=12, mode="auto")
    model.fill_random(1234)
    sm = dn.apply_streaming(model, device=dev, prefetch_slots=2, profile=False)
    _log(f"streaming: {n_blocks} blocks captured into pinned memory in {time.perf_counter() - t:.1f} s")
    g = torch.Generator().manual_seed(99)
    x = torch.randn((1, 4096, 5120), generator=g).to(torch.bfloat16).to(dev)
    ctx = torch.randn((1, 512, 5120), generator=g).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        ms = _timed(torch, lambda: sm(x, ctx), steps, 1)
        sm.state.profiler = prof_mod._StreamProfiler(n_blocks, sm.state.flat_bytes, True)
        for _ in range(3):
            y_stream = sm(x, ctx)
    torch.cuda.synchronize()
    prof = sm.profile_summary()["mean_excluding_first_forward"]
    flat = sm.state.flat_bytes
    # the link's own rate: block 0's pinned host flat into slot 0, five copies alone on the copy stream
    st = sm.state
    a, b = native.Event(timing=True), native.Event(timing=True)
    a.record(st.prefetch_stream.handle)
    for _ in range(5):
        native.call("wf_h2d_async", st.slot_flats[0].data_ptr(), st.host_flats[0].data_ptr(), flat,
                    st.prefetch_stream.handle)
    b.record(st.prefetch_stream.handle)
    b.synchronize()
    raw_ms = a.elapsed_ms(b) / 5
    identical = _resident_check(torch, sm, model, x, ctx, y_stream, dev)
    del model, sm
    torch.cuda.empty_cache()
    return {"ms_per_step": round(ms, 2), "blocks": n_blocks, "slots": 2, "bytes_per_block": flat,
            "bit_identical_to_resident": identical,
            "h2d_GBps_effective": round(flat * n_blocks / (ms / 1e3) / 1e9, 2),
            "raw_h2d_GBps": round(flat / (raw_ms / 1e3) / 1e9, 2),
            "copy_floor_ms_per_step": round(n_blocks * raw_ms, 1),
            "profiled": {"forward_ms": prof["forward_ms"], "dma_ms": prof["dma_ms"], "stall_ms": prof["stall_ms"],
                         "compute_ms": prof["streamed_compute_ms"],
                         "hidden_fraction": prof["overlap_ratio"], "dma_gbps": prof["dma_gbps"],
                         "hidden_fraction_bound": round(min(1.0, prof["streamed_compute_ms"] / prof["dma_ms"]), 4)},
            "linears": "GGUFLinear mode auto: wf_dequant + wf_linear_bf16 at 4096 rows, the fused panel form at 512 rows"}


def chunk_leg(torch, native, n_blocks=40, steps=5, chunk_mb=96, slots=4):
    """Chunk (sub-block) streaming of the same 40 blocks: the GPU holds ``slots`` chunks of at most ``chunk_mb`` MB of
    a block's linears (plus a spare) instead of two whole blocks. The first forward learns the call order (each
    linear copied on the compute stream just before it runs); the timed forwards stream chunk units."""
    syn = importlib.import_module(PKG + ".streaming.synthetic")
    dn = importlib.import_module(PKG + ".streaming.dit_node")
    dev = torch.device("cuda:0")
    model = syn.WanLikeStack(n_blocks=n_blocks, qtype=12, mode="auto")
    model.fill_random(1234)
    sm = dn.apply_streaming(model, device=dev, chunk=True, chunk_bytes=chunk_mb * 1024 ** 2, chunk_slots=slots)
    g = torch.Generator().manual_seed(99)
    x = torch.randn((1, 4096, 5120), generator=g).to(torch.bfloat16).to(dev)
    ctx = torch.randn((1, 512, 5120), generator=g).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        torch.cuda.synchronize()
        t = time.perf_counter()
        sm(x, ctx)
        torch.cuda.synchronize()
        calib_ms = (time.perf_counter() - t) * 1e3
        ms = _timed(torch, lambda: sm(x, ctx), steps, 1)
        y_stream = sm(x, ctx)
    st = sm.state
    res = {"ms_per_step": round(ms, 2), "calibration_forward_ms": round(calib_ms, 1), "blocks": n_blocks,
           "chunk_mb": chunk_mb, "slots": slots, "chunks_per_block": st.n_types,
           "chunk_slot_bytes": st.slot_bytes, "gpu_weight_bytes": st.slot_bytes * (slots + len(st.spares)),
           "block_mode_gpu_weight_bytes": 2 * st.flat_bytes, "spare_uses": st.spare_uses,
           "h2d_GBps_effective": round(st.flat_bytes * n_blocks / (ms / 1e3) / 1e9, 2)}
    res["bit_identical_to_resident"] = _resident_check(torch, sm, model, x, ctx, y_stream, dev)
    del model, sm
    torch.cuda.empty_cache()
    return res


def ssd_leg(torch, native, n_blocks=40, ram_blocks=20, steps=3):
    """SSD tier: 40 Wan-14B blocks (Q4_K, 197.7 MB each) written as a GGUF model file to local disk
    (WEIGHTFERRY_SSD_DIR, else the temp directory); the native ring's raw O_DIRECT read rate over the whole file with
    1, 2 and 4 reader threads (4 pinned buffers), then a streamed forward (4096 tokens) with ``ram_blocks`` blocks in
    pinned RAM and the others (interleaved) read from the file on every step through the ring (4 buffers, 2 readers)."""
    import tempfile
    syn = importlib.import_module(PKG + ".streaming.synthetic")
    dn = importlib.import_module(PKG + ".streaming.dit_node")
    src = importlib.import_module(PKG + ".core.tiers.sources")
    common = importlib.import_module(PKG + ".streaming.common")
    dev = torch.device("cuda:0")
    path = os.path.join(os.environ.get("WEIGHTFERRY_SSD_DIR") or tempfile.gettempdir(), f"wf_ssd_{os.getpid()}.gguf")
    model = syn.WanLikeStack(n_blocks=n_blocks, qtype=12, mode="dequant")
    model.fill_random(1234)
    t = time.perf_counter()
    syn.write_gguf_model(model, path)
    with open(path, "rb") as f:
        os.fsync(f.fileno())
    size = os.path.getsize(path)
    _log(f"ssd: wrote {size / 1e9:.2f} GB GGUF in {time.perf_counter() - t:.1f} s")
    try:
        offsets, flat_bytes = common._flat_layout(common._specs(model.blocks[0]))
        pnames = [n for n, _ in model.blocks[0].named_parameters()]
        source, _ = src.gguf_block_source(path, [[f"blocks.{i}.{p}" for p in pnames] for i in range(n_blocks)],
                                          offsets)
        block_bytes = source.block_bytes
        reads = {}
        for threads in (1, 2, 4):
            ring = src.DiskRing(source, depth=4, pin=True, threads=threads, direct=True, device=dev)
            t0 = time.perf_counter()
            for b in range(n_blocks):
                _, slot = ring.acquire(b)
                ring.release(slot)
            dt = time.perf_counter() - t0
            ring.close()
            reads[f"threads_{threads}_GBps"] = round(block_bytes * n_blocks / dt / 1e9, 2)
        _log(f"ssd: ring reads {reads}")
        g = torch.Generator().manual_seed(99)
        x = torch.randn((1, 4096, 5120), generator=g).to(torch.bfloat16).to(dev)
        ctx = torch.randn((1, 512, 5120), generator=g).to(torch.bfloat16).to(dev)
        sm = dn.apply_streaming(model, device=dev, prefetch_slots=2, profile=False, model_file=path,
                                ram_blocks=ram_blocks, ring_depth=4, ring_threads=2)
        n_disk = len(sm.state.disk_index)
        with torch.no_grad():
            ms = _timed(torch, lambda: sm(x, ctx), steps, 1)
            y_stream = sm(x, ctx)
        st = sm.state.ring.stats()
        identical = _resident_check(torch, sm, model, x, ctx, y_stream, dev)
    finally:
        os.remove(path)
    del model
    torch.cuda.empty_cache()
    return {"file_GB": round(size / 1e9, 3), "ring_raw_read": reads, "ms_per_step": round(ms, 1),
            "bit_identical_to_resident": identical,
            "blocks": n_blocks, "ram_tier_blocks": n_blocks - n_disk, "ssd_tier_blocks": n_disk,
            "ssd_bytes_per_step": block_bytes * n_disk,
            "ssd_GBps_per_step": round(block_bytes * n_disk / (ms / 1e3) / 1e9, 2),
            "ring_reads": st["reads"], "layout": "interleave", "direct_io": True}


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def lora_leg(torch, native, raw, shape, steps=20):
    """wf_dequant_add on one Q4_K weight (MID float16 -> bf16): the first LoRA inside the dequantisation (blocks +
    float32 difference in, bf16 out) and a later LoRA onto the weight (bf16 + difference in, bf16 out). Two copies
    of every buffer alternate (1.2 GB in all), so the last-level cache does not serve a call's bytes to the next."""
    lib = native.lib()
    dev = torch.device("cuda:0")
    stream = native.stream_of(dev)
    n = shape[0] * shape[1]
    g = torch.Generator(device=dev).manual_seed(1234)
    bufs = [(torch.from_numpy(raw).to(dev), torch.randn(n, generator=g, device=dev) * 0.01,
             torch.empty(n, dtype=torch.bfloat16, device=dev)) for _ in range(2)]
    res = {}
    for name, first in (("first_lora_fused_into_dequant", True), ("later_lora_onto_weight", False)):
        turn = [0]

        def call():
            rw, df, out = bufs[turn[0] % 2]
            turn[0] += 1
            rc = lib.wf_dequant_add(rw.data_ptr() if first else None, rw.numel() if first else 0, 12, 0, 1,
                                    df.data_ptr(), 0.5, out.data_ptr(), n, stream)
            if rc != 0:
                raise RuntimeError(native.last_error())
        ms = _timed(torch, call, steps, 3)
        nbytes = (raw.size + 4 * n + 2 * n) if first else (2 * n + 4 * n + 2 * n)
        res[name] = {"GB/s": round(nbytes / (ms / 1e3) / 1e9, 1), "kernel_us": round(ms * 1e3, 1),
                     "frac": round(nbytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 3), "bytes": nbytes}
    del bufs
    torch.cuda.empty_cache()
    return res


def dequant_leg(torch, native, raws, shapes, qtype, mid, out_dt, steps, warmup):
    """Time `steps` steps of dequantising every matrix once, launched back to back on torch's current stream with
    events at both ends of the timed region on that stream. Returns (ms per step, mean ms per launch, bytes/step);
    the launches are all of one kernel, so the mean per launch is that kernel's average duration. Steps cycle over
    at least ROTATE copies of inputs and outputs and at least ROTATE_BYTES in all, so the last-level cache (256 MB)
    cannot serve one step's bytes to a later one."""
    lib = native.lib()
    dev = torch.device("cuda:0")
    stream = native.stream_of(dev)
    out_torch = {0: torch.float16, 1: torch.bfloat16, 2: torch.float32}[out_dt]
    nvals = [s[0] * s[1] for s in shapes]
    algo = sum(r.size for r in raws) + sum(n * torch.empty((), dtype=out_torch).element_size() for n in nvals)
    rot = max(ROTATE, -(-ROTATE_BYTES // algo))
    ins = [[torch.from_numpy(r).to(dev) for r in raws] for _ in range(rot)]
    outs = [[torch.empty(s, dtype=out_torch, device=dev) for s in shapes] for _ in range(rot)]

    def launch(r, m):
        rc = lib.wf_dequant(ins[r][m].data_ptr(), ins[r][m].numel(), qtype, mid, out_dt, outs[r][m].data_ptr(),
                            nvals[m], stream)
        if rc != 0:
            raise RuntimeError(native.last_error())

    turn = [0]

    def one_step():
        turn[0] += 1
        for m in range(len(shapes)):
            launch(turn[0] % rot, m)
    _warm_clock(torch, one_step)
    for i in range(warmup):
        for m in range(len(shapes)):
            launch(i % rot, m)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        for m in range(len(shapes)):
            launch(i % rot, m)
    t1.record()
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / steps
    del ins, outs
    torch.cuda.empty_cache()
    return ms_step, ms_step / len(shapes), algo


def probe_lib():
    """libwf_probe.so, the byte-moving kernel the ceiling leg runs (measurement only: built from csrc/probe/ beside
    the product library, never part of it)."""
    import ctypes
    path = os.path.join(ROOT, PKG, "lib", "libwf_probe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (make -C {PKG}/csrc)")
    lib = ctypes.CDLL(path)
    p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.wfp_hbm_stream.argtypes, lib.wfp_hbm_stream.restype = [p, p, i64, i32, i32, p], i32
    lib.wfp_last_error.argtypes, lib.wfp_last_error.restype = [], ctypes.c_char_p
    return lib


def hbm_stream_leg(torch, native, nbytes, reads, writes, steps, warmup):
    """What HBM delivers to a kernel that only moves bytes (wfp_hbm_stream: reads:writes 16-byte chunks per thread,
    non-temporal stores) for about `nbytes` per launch, with the dequant legs' rotation over ROTATE_BYTES. Returns
    (bytes per launch, mean us per launch)."""
    lib = probe_lib()
    dev = torch.device("cuda:0")
    stream = native.stream_of(dev)
    items = nbytes // (16 * (reads + writes))
    per = 16 * items * (reads + writes)
    rot = max(ROTATE, -(-ROTATE_BYTES // per))
    ins = [torch.empty(max(16, 16 * items * reads), dtype=torch.uint8, device=dev) for _ in range(rot)]
    outs = [torch.empty(max(16, 16 * items * writes), dtype=torch.uint8, device=dev) for _ in range(rot)]
    for t in ins:
        t.fill_(1)

    def launch(r):
        rc = lib.wfp_hbm_stream(ins[r].data_ptr(), outs[r].data_ptr(), items, reads, writes, stream)
        if rc != 0:
            raise RuntimeError(lib.wfp_last_error().decode())

    for i in range(warmup):
        launch(i % rot)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        launch(i % rot)
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / steps
    del ins, outs
    torch.cuda.empty_cache()
    return per, us


# the dequantisation launches set beside a byte-moving kernel of the same size and nearest read:write mix
CEILINGS = (("q4_k_13824x5120_mix_2_7", 181_370_880, 2, 7), ("q8_0_5120sq_mix_1_2", 80_281_600, 1, 2),
            ("q4_0_5120sq_mix_2_7", 67_174_400, 2, 7), ("q6_k_5120sq_mix_1_2", 73_932_800, 1, 2))


def ceiling_leg(torch, native, steps, warmup):
    res = {}
    for name, nbytes, r, w in CEILINGS:
        per, us = hbm_stream_leg(torch, native, nbytes, r, w, steps, warmup)
        res[name] = {"GB/s": round(per / us / 1e3, 1), "kernel_us": round(us, 2), "bytes": per,
                     "frac": round(per / us / 1e3 / HBM_PEAK_GBS, 3)}
    return res


FORMATS = ((2, "q4_0"), (3, "q4_1"), (6, "q5_0"), (7, "q5_1"), (13, "q5_k"), (14, "q6_k"), (10, "q2_k"),
           (11, "q3_k"))


def formats_leg(torch, native, encode, steps, warmup):
    """Dequantisation of one 5120 x 5120 weight in each remaining GGML format -> bf16 (MID float16): GB/s of the
    algorithmic bytes (blocks in + bf16 out) over the mean launch, and the fraction of the HBM peak."""
    shape = (5120, 5120)
    w = encode.weights(shape, seed=1234)
    res = {}
    for qt, name in FORMATS:
        if qt in encode.ENCODERS:
            raw = encode.encode(w, qt)
        else:
            raw = encode.random_blocks(qt, shape[0] * shape[1] // encode.PER_BLOCK[qt], seed=1234)
        _, k, a = dequant_leg(torch, native, [raw], [shape], qt, 0, 1, steps, warmup)
        res[name] = {"GB/s": round(a / (k / 1e3) / 1e9, 1), "kernel_us": round(k * 1e3, 2),
                     "frac": round(a / (k / 1e3) / 1e9 / HBM_PEAK_GBS, 3), "bytes": a}
    return res


def _cpu_host(torch):
    """Threads for the CPU legs and what the host is: torch takes every CPU this process may use -- os.cpu_count(),
    bounded by the process's CPU affinity, its cgroup CPU quota and OMP_NUM_THREADS where the host sets one (a
    shared host's statement of this process's CPU share; more threads than that share only contend). Returns the
    fields each cpu_baseline record carries."""
    nproc = os.cpu_count() or 1
    share, why = nproc, ["os.cpu_count()"]
    try:
        aff = len(os.sched_getaffinity(0))
        if aff < share:
            share, why = aff, ["CPU affinity"]
    except (AttributeError, OSError):
        pass
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            q = max(1, -(-int(quota) // int(period)))
            if q < share:
                share, why = q, ["cgroup cpu.max"]
    except (OSError, ValueError):
        pass
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and 0 < int(omp) < share:
        share, why = int(omp), ["OMP_NUM_THREADS"]
    torch.set_num_threads(share)
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cores": torch.get_num_threads(), "nproc": nproc, "threads_bound_by": why[0], "cpu_model": model}


def cpu_baseline_dequant(torch, raw, qtype, rows, cols, budget_s=12.0):
    """The reference's CPU path (ComfyUI-GGUF's torch op chain, restated in oracle.torch_chain) on the first
    `rows` rows of one weight; GB/s with the same byte accounting as the GPU leg."""
    from oracle import torch_chain
    ts = torch_chain.TYPE_SIZE[qtype]
    per = torch_chain.BLOCK_SIZE[qtype]
    nbytes = rows * cols // per * ts
    sample = torch.from_numpy(raw[:nbytes].copy())
    host = _cpu_host(torch)
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
    return {"value": round(algo / med / 1e9, 3), "unit": "GB/s", **host, "kind": "port",
            "sample": f"ComfyUI-GGUF torch op chain (oracle/torch_chain.py) on CPU, Q4_K -> bf16 (MID f16), "
                      f"first {rows} of the 13824 rows of the 13824x5120 weight ({nbytes} bytes in, "
                      f"{rows * cols * 2} out; GB/s is size-independent for this streaming op), median of "
                      f"{len(times)} runs"}


def _cpu_median(fn, budget_s, runs=10):
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < runs and time.perf_counter() < t_end:
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baselines(torch, encode):
    """The reference's CPU path beside every other workload row, each on a bounded sample (a few seconds): ComfyUI-
    GGUF's torch op chain (oracle/torch_chain.py) for the dequantisation, torch's bf16 F.linear after it, and
    torch._int_mm with the scale epilogue for the int8 linear; the streamed forward has no CPU path in the reference,
    so its baseline is the CPU dequantisation + linear of one Wan block, extrapolated to 4096 tokens x 40 blocks."""
    from oracle import torch_chain
    host = _cpu_host(torch)
    res = {}
    # Q8_0, first 512 rows of the 5120 x 5120 weight
    raw = encode.encode_q8_0(encode.weights((512, 5120), seed=1234))
    t8 = torch.from_numpy(raw)
    med, n = _cpu_median(lambda: torch_chain.dequantize(t8, 8, (512, 5120), torch.float16, torch.bfloat16), 6.0)
    res["q8_0_dequant"] = {"value": round((raw.size + 512 * 5120 * 2) / med / 1e9, 3), "unit": "GB/s", **host,
                           "kind": "port", "sample": f"Q8_0 -> bf16 (MID f16), 512 rows x 5120, median of {n}"}
    # fused-GEMM row: Q5_K dequantisation of one 5120 x 5120 layer + bf16 F.linear at 64 tokens
    raw5 = torch.from_numpy(encode.random_blocks(13, 5120 * 5120 // 256, seed=1234))
    x = torch.randn((64, 5120)).to(torch.bfloat16)

    def layer():
        w = torch_chain.dequantize(raw5, 13, (5120, 5120), torch.float16, torch.bfloat16)
        return torch_chain.linear_bf16(x, w)
    med, n = _cpu_median(layer, 8.0, 5)
    res["q5_k_dequant_plus_linear"] = {"value": round(2 * 64 * 5120 * 5120 / med / 1e12, 4), "unit": "TFLOPS",
                                       **host, "kind": "port", "ms_per_layer": round(med * 1e3, 1),
                                       "sample": f"Q5_K 5120x5120 dequant + bf16 linear, 64 tokens, median of {n}"}
    # int8 W8A8 row: torch._int_mm + (acc * xs) * ws epilogue, 256 x 5120 by 5120 x 5120
    xq = torch.randint(-127, 128, (256, 5120), dtype=torch.int8)
    wq = torch.randint(-127, 128, (5120, 5120), dtype=torch.int8)
    wqt = wq.t().contiguous()
    xs, ws = torch.rand(256) * 0.01, torch.rand(5120) * 0.01

    def i8():
        acc = torch._int_mm(xq, wqt)
        return ((acc.float() * xs[:, None]) * ws[None, :]).to(torch.bfloat16)
    med, n = _cpu_median(i8, 6.0)
    res["int8_linear"] = {"value": round(2 * 256 * 5120 * 5120 / med / 1e12, 4), "unit": "TOPS", **host,
                          "kind": "port", "sample": f"torch._int_mm 256x5120 by 5120x5120 + scale epilogue, median of {n}"}
    # streamed row: one Wan block's linears (Q4_K) on the CPU at 64 tokens -- eight 5120 x 5120 layers and two of
    # 13824 x 5120 elements (ffn up / down), timed once per shape on random blocks; the dequantisations (per call,
    # not per token) counted once, the GEMMs scaled to 4096 tokens; x 40 blocks
    t_deq = t_mm = 0.0
    for (N, K), count in (((5120, 5120), 8), ((13824, 5120), 2)):
        r = torch.from_numpy(encode.random_blocks(12, N * K // 256, seed=N))
        xb = torch.randn((64, K)).to(torch.bfloat16)
        dq, _ = _cpu_median(lambda: torch_chain.dequantize(r, 12, (N, K), torch.float16, torch.bfloat16), 2.0, 3)
        w = torch_chain.dequantize(r, 12, (N, K), torch.float16, torch.bfloat16)
        mm, _ = _cpu_median(lambda: torch_chain.linear_bf16(xb, w), 2.0, 3)
        t_deq += count * dq
        t_mm += count * mm
    block_s = t_deq + t_mm * 4096 / 64
    res["streamed_block_linears"] = {"value": round(40 * block_s * 1e3, 0), "unit": "ms/step (extrapolated)",
                                     **host, "kind": "port",
                                     "sample": "one Wan block's 10 Q4_K linears on the CPU: dequantisation "
                                               f"{t_deq * 1e3:.0f} ms + bf16 GEMMs at 64 tokens {t_mm * 1e3:.0f} ms "
                                               "scaled to 4096 tokens, x 40 blocks (linears only; attention "
                                               "excluded)"}
    return res


def _traffic():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3 counter summary (FETCH_SIZE +
    WRITE_SIZE scaled by the plain-copy calibration), or None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "dequant_q4_k_ffn_pmc.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def main():
    args = _args()
    if args.gpus != 1:
        print(f"bench.py: runs on one GPU; --gpus {args.gpus} is not supported "
              "(the one-GPU throughput is the reported value)", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, ROOT)
    import numpy as np  # noqa: F401
    import torch

    encode = importlib.import_module(PKG + ".gguf_encode")

    native = importlib.import_module(PKG + "._native")
    native.lib()
    _log(f"library {native.LIB_PATH}")

    shapes = [(13824, 5120), (5120, 13824)]
    also = {}
    raws = None
    if args.legs & {"headline", "lora"}:
        t = time.perf_counter()
        raws = [encode.encode_q4_k(encode.weights(s, seed=1234 + i)) for i, s in enumerate(shapes)]
        _log(f"encoded Q4_K pair in {time.perf_counter() - t:.1f} s")
    if "headline" not in args.legs:
        if "ceiling" in args.legs:
            also["hbm_stream_same_mix"] = ceiling_leg(torch, native, args.steps, args.warmup)
        if "formats" in args.legs:
            also["dequant_formats_5120sq"] = formats_leg(torch, native, encode, args.steps, args.warmup)
        if "lora" in args.legs:
            also["lora_add_q4_k_13824x5120"] = lora_leg(torch, native, raws[0], shapes[0])
        if "int8" in args.legs:
            also["int8_w8a8"] = int8_leg(torch, native)
        if "fused" in args.legs:
            also["fused_dequant_gemm_wan_block"] = fused_leg(torch, native)
        if "streaming" in args.legs:
            also["streamed_40_blocks_q4_k"] = streaming_leg(torch, native)
        if "chunk" in args.legs:
            also["chunk_streamed_40_blocks_q4_k"] = chunk_leg(torch, native)
        if "ssd" in args.legs:
            also["ssd_tier_40_blocks_q4_k"] = ssd_leg(torch, native)
        print(json.dumps({"legs": sorted(args.legs), "also": also}), flush=True)
        return

    ms_step, kern_ms, algo = dequant_leg(torch, native, raws, shapes, 12, 0, 1, args.steps, args.warmup)
    value = algo / (ms_step / 1e3) / 1e9
    per_launch = algo / len(shapes)
    achieved = per_launch / (kern_ms / 1e3) / 1e9
    _log(f"Q4_K pair: {ms_step * 1e3:.1f} us/step, kernel {kern_ms * 1e3:.1f} us, {value:.0f} GB/s")

    # calibration: a plain copy of 512 MiB (two rotating pairs: 2 GiB in all) -- the achievable HBM rate, and the
    # known-size kernel the counter runs are scaled by
    cp = [(torch.empty(1 << 29, dtype=torch.uint8, device="cuda"), torch.empty(1 << 29, dtype=torch.uint8,
                                                                               device="cuda")) for _ in range(2)]
    turn = [0]

    def copy_once():
        src, dst = cp[turn[0] % 2]
        turn[0] += 1
        dst.copy_(src)
    ms_cp = _timed(torch, copy_once, 10, 2)
    also["plain_copy_512MiB"] = {"GB/s": round(2 * (1 << 29) / ms_cp / 1e6, 1), "us": round(ms_cp * 1e3, 1)}
    del cp
    torch.cuda.empty_cache()
    # MID float32 on the same pair
    ms32, k32, _ = dequant_leg(torch, native, raws, shapes, 12, 2, 1, max(5, args.steps // 2), 3)
    also["q4_k_pair_mid_f32"] = {"GB/s": round(algo / (ms32 / 1e3) / 1e9, 1),
                                 "kernel_us": round(k32 * 1e3, 2)}
    # Q8_0 5120 x 5120 (MID float16 and float32 -> bf16), and the 14B-DiT FFN pair in Q8_0
    q8 = [encode.encode_q8_0(encode.weights((5120, 5120), seed=1234))]
    for mid, name in ((0, "q8_0_5120sq_mid_f16"), (2, "q8_0_5120sq_mid_f32")):
        ms8, k8, a8 = dequant_leg(torch, native, q8, [(5120, 5120)], 8, mid, 1, args.steps, args.warmup)
        also[name] = {"GB/s": round(a8 / (k8 / 1e3) / 1e9, 1), "kernel_us": round(k8 * 1e3, 2),
                      "frac": round(a8 / (k8 / 1e3) / 1e9 / HBM_PEAK_GBS, 3), "bytes": a8}
    q8p = [encode.encode_q8_0(encode.weights(sh, seed=1234 + i)) for i, sh in enumerate(shapes)]
    ms8, k8, a8 = dequant_leg(torch, native, q8p, shapes, 8, 0, 1, args.steps, args.warmup)
    also["q8_0_ffn_pair_mid_f16"] = {"GB/s": round(a8 / (ms8 / 1e3) / 1e9, 1), "kernel_us": round(k8 * 1e3, 2),
                                     "frac": round(a8 / (ms8 / 1e3) / 1e9 / HBM_PEAK_GBS, 3), "bytes": a8}
    del q8p
    if "ceiling" in args.legs:
        ceil = ceiling_leg(torch, native, args.steps, args.warmup)
        also["hbm_stream_same_mix"] = ceil
        also["q8_0_5120sq_mid_f16"]["of_same_mix_stream"] = round(
            also["q8_0_5120sq_mid_f16"]["GB/s"] / ceil["q8_0_5120sq_mix_1_2"]["GB/s"], 3)
        also["q4_k_13824x5120_of_same_mix_stream"] = round(achieved / ceil["q4_k_13824x5120_mix_2_7"]["GB/s"], 3)
        _log("ceiling leg done")
    if "formats" in args.legs:
        also["dequant_formats_5120sq"] = formats_leg(torch, native, encode, args.steps, args.warmup)
        _log("formats leg done")
    if "lora" in args.legs:
        also["lora_add_q4_k_13824x5120"] = lora_leg(torch, native, raws[0], shapes[0])
        _log("lora leg done")
    if "int8" in args.legs:
        also["int8_w8a8"] = int8_leg(torch, native)
        _log("int8 leg done")
    if "fused" in args.legs:
        also["fused_dequant_gemm_wan_block"] = fused_leg(torch, native)
        _log("fused leg done")
    if "streaming" in args.legs:
        also["streamed_40_blocks_q4_k"] = streaming_leg(torch, native)
        _log("streaming leg done")
    if "chunk" in args.legs:
        also["chunk_streamed_40_blocks_q4_k"] = chunk_leg(torch, native)
        _log("chunk leg done")
    if "ssd" in args.legs:
        also["ssd_tier_40_blocks_q4_k"] = ssd_leg(torch, native)
        _log("ssd leg done")
    cpu = None
    if not args.skip_cpu:
        cpu = cpu_baseline_dequant(torch, raws[0], 12, 512, 5120)
        _log(f"cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads")
        also["cpu_baselines"] = cpu_baselines(torch, encode)
        _log("cpu baselines of the other rows done")

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
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": _traffic(),
                     "kernel": "wf::deq_items<wf::Q45_K<12, f16, bf16>>", "kernel_us": round(kern_ms * 1e3, 2),
                     "bytes_per_launch": per_launch},
        "cpu_baseline": cpu,
        "also": also,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
