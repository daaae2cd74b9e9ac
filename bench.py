"""Benchmark of the TSAC probability model on one MI355X.

Step = one GPU encode (pack_normal-equivalent: model + range coder -> FBAZ
bytes) plus one GPU decode (unpack_normal-equivalent: model + range decoder ->
tokens, CRC checked) of a 30 s joint-stereo token stream: 2580 frames x 12
codebooks, entropy batch 3 (three lanes of 860 frames), one channel group, on
the probability model of 12 temporal + 3 codebook layers, width 1024, 16 x 64
heads, FFN 4096, with seeded random-init weights in the reference's packed
layout. Tokens are synthetic (uniform over the 1024-symbol alphabet).
`--geometry reference` runs the reference's own geometry (width 512, 4 x 128
heads, FFN 2048) instead; by default that geometry is measured as the
secondary `reference_geometry` entry.

value = tokens / (encode seconds + decode seconds) of one step, with the
session-timed host-to-device copies of the calls' inputs taken out.

Also measured in the same run:
  * roofline: the timed region's dominant kernel, the decode frame step
    (frame_kernel, up to 64 steps per launch, ~98% of the round trip): algorithmic
    bytes per step (every projection's int8 weights, block scales and bias
    once per step, plus the lanes' temporal key/value cache rows at the
    average context position) over the average step time, measured with HIP
    events around the step loop on the session's own stream (the stream the
    kernel is launched on). It is bound by the latency of its ~240 dependent
    jobs, not by HBM. `traffic` is the HBM bytes per step recorded by the
    calibrated rocprofv3 PMC runs named in `traffic_source` (not measured in
    this run).
  * roofline_gemv: the decode GEMV streaming int8 weights from HBM: K=1024,
    M=3 columns, 4 distinct 256 MiB weight matrices (1 GiB, larger than the
    256 MB MALL) rotated across launches; HIP events on the launch stream.
  * roofline_gemm: the encode MFMA GEMM on the codebook-stack qkv shape
    (M = 30,960 rows, K = 512, N = 1536).
  * qlinear: the isolated quantized linear (K=1024, N in {1024, 4096},
    M in {1, 3, 64, 1024, 4096}). For M <= 64 each launch reads a different
    weight matrix, rotating through >= 1 GiB of distinct matrices inside one
    captured HIP graph (so the weights stream from HBM, not the 256 MB MALL);
    per-launch time = graph time / launches.
  * reference_geometry: the same round trip on the reference geometry
    (width 512, 4 x 128 heads, FFN 2048), 2580 frames, batch 3, with its own
    frame-step roofline.
  * token_stream_round_trip_s: the step's encode + decode seconds (30 s of
    audio as tokens). encode_decode_s_per_30s_stereo is the PCM round trip of
    30 s of joint-stereo audio (DAC analysis, RVQ, model and range coding, then
    back to PCM), from `end_to_end`.
  * attention: causal multi-head attention alone (16 x 64 heads, batch 3,
    T in {256, 1290, 2580}): causal prefill TFLOP/s and one-query decode GB/s.
  * attainable: this device's streaming-read rate and int8 MFMA rate, measured
    by the library's calibration kernels; each roofline also reports its
    fraction of these.
  * cpu_baseline: the C oracle (bit-exact restatement of the reference CPU
    path, lane-parallel like the reference's executor): encode + decode round
    trip of a bounded sample (1290 frames, 15 s of audio), same rate definition.
"""
import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for path in (ROOT, ROOT / "tsac-metal_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

import numpy as np  # noqa: E402

HBM_PEAK_GBPS = 8000.0
INT8_PEAK_TOPS = 5000.0
FP32_PEAK_TFLOPS = 157.3


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--frames", type=int, default=2580)
    p.add_argument("--batch", type=int, default=3)
    p.add_argument("--geometry", choices=["reference", "wide"], default="wide")
    p.add_argument("--only", choices=["all", "model", "gemv", "gemm", "attention", "qlinear", "reference", "audio"],
                   default="all")
    p.add_argument("--gemv-launches", type=int, default=64)
    p.add_argument("--cpu-frames", type=int, default=0,
                   help="CPU baseline sample in frames (default: 1290 at the reference geometry, 430 at the wide one)")
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


def gemv_roofline(torch, native, launches):
    """Decode GEMV streaming 1 GiB of distinct int8 weights (K=1024, M=3)."""
    K, M, rows, mats = 1024, 3, 262144, 4
    rng = np.random.default_rng(17)
    linears = []
    for i in range(mats):
        values = np.frombuffer(rng.bytes(rows * K), np.int8).reshape(rows, K)
        values = np.where(values == -128, np.int8(-127), values)  # int8 in [-127, 127]
        scales = np.full((K // 256, rows), 0.0078125, np.float32)
        bias = np.zeros(rows, np.float32)
        linears.append(native.DeviceLinear(values, scales, bias))
        del values
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    xb = (x.view(torch.int32) >> 16).to(torch.int16).contiguous()
    q = torch.empty((M, K), dtype=torch.int8, device="cuda")
    s = torch.empty((M, K // 256), dtype=torch.float32, device="cuda")
    native.bf8l(xb, M, K, q, s)
    y = torch.empty((M, rows), dtype=torch.int16, device="cuda")
    for i in range(8):
        linears[i % mats].apply_quantized(q, s, M, y, path=native.PATH_GEMV)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(launches):
        linears[i % mats].apply_quantized(q, s, M, y, path=native.PATH_GEMV)
    stop.record()
    torch.cuda.synchronize()
    seconds = start.elapsed_time(stop) / 1000 / launches
    traffic = K * rows + 16 * rows + 4 * rows + M * K + M * (K // 256) * 4 + 2 * M * rows
    achieved = traffic / seconds / 1e9
    del linears
    torch.cuda.empty_cache()
    # Calibration for hardware byte counters: a plain 256 MiB device copy.
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    measured, source = recorded_traffic("gemv_rotating_1GiB_K1024_M3.traffic.txt", "bytes_per_launch")
    return {"kernel": "gemv_kernel<3>", "bound": "hbm", "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured, "traffic_source": source, "bytes_per_launch": traffic,
            "avg_launch_us": round(seconds * 1e6, 2),
            "shape": {"K": K, "N": rows, "M": M, "distinct_weight_bytes": mats * rows * K}}


def recorded_traffic(name, field):
    """HBM bytes per launch recorded in profiles/<name> from two calibrated
    rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE) of the same workload;
    this run does not measure them. Returns (bytes or None, source label)."""
    record = ROOT / "profiles" / name
    if not record.exists():
        return None, None
    fields = dict(line.split("=", 1) for line in record.read_text().split() if "=" in line)
    return int(float(fields[field])), f"recorded in profiles/{name} (rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE, " \
                                      f"calibrated against a device copy); not measured in this run"


def calibration_copy(torch, mib=256):
    """One plain device-to-device copy of `mib` MiB: under rocprofv3 --pmc its
    FETCH_SIZE and WRITE_SIZE give the factors that turn those counters into
    bytes on this hardware (the copy reads and writes exactly mib MiB)."""
    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def attainable_peaks(torch, native):
    """Attainable rates on this device: a streaming read of 4 rotating 256 MiB
    buffers with the GEMV's load pattern, and independent int8 MFMA chains."""
    buffers = [torch.empty(256 << 20, dtype=torch.uint8, device="cuda") for _ in range(4)]
    for b in buffers:
        b.fill_(1)
    stream = torch.cuda.current_stream()
    for i in range(16):
        native.probe_read(buffers[i % 4], stream)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    launches = 64
    read = 0.0
    for _ in range(3):
        start.record(stream)
        for i in range(launches):
            native.probe_read(buffers[i % 4], stream)
        stop.record(stream)
        torch.cuda.synchronize()
        read = max(read, (256 << 20) * launches / (start.elapsed_time(stop) / 1000) / 1e9)
    del buffers
    torch.cuda.empty_cache()
    native.probe_mfma(4096, 4000, stream)
    mfma = 0.0
    for _ in range(3):
        start.record(stream)
        ops = native.probe_mfma(4096, 4000, stream)
        stop.record(stream)
        torch.cuda.synchronize()
        mfma = max(mfma, ops / (start.elapsed_time(stop) / 1000) / 1e12)
    # A probe that beats the published peaks did not do its work.
    assert read < 1.05 * HBM_PEAK_GBPS and mfma < 1.05 * INT8_PEAK_TOPS, (read, mfma)
    return {"hbm_read_GBps": round(read, 1), "int8_mfma_TOPs": round(mfma, 1),
            "method": "probe_read (16-byte nontemporal loads, 64 KiB per workgroup, 1 GiB rotating) and "
                      "probe_mfma (4096 x 4 waves, 4 independent v_mfma_i32_32x32x32_i8 chains)"}


def gemm_roofline(torch, native, launches=20):
    """Encode MFMA GEMM on operand-tile activations (the encode's layout) for the
    codebook stack's projections at M = 2580*12 rows; the first shape (qkv) is
    the headline, the rest are listed with their rates. HIP events on the
    launch stream (the default stream, as torch's events)."""
    from tsac_hip.synthetic import random_linear

    shapes = [(30960, 512, 1536, False), (30960, 512, 512, True), (30960, 512, 2048, False),
              (30960, 2048, 512, True), (30960, 512, 1024, False)]
    rng = np.random.default_rng(23)
    rows = []
    for M, K, N, with_residual in shapes:
        linear = native.DeviceLinear(*random_linear(rng, K, N))
        P = native.tile_rows(M)
        x = torch.from_numpy(np.ascontiguousarray(
            (rng.standard_normal((M, K)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.int16)))
        x = x.cuda()
        q = torch.empty(P * K, dtype=torch.int8, device="cuda")
        s = torch.empty(K // 256 * P, dtype=torch.float32, device="cuda")
        native.bf8l_tiles(x, M, K, q, s)
        y = torch.zeros((M, N), dtype=torch.int16, device="cuda")
        residual = y if with_residual else None
        for _ in range(3):
            linear.apply_quantized(q, s, M, y, residual=residual, path=native.PATH_GEMM_TILES)
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(launches):
            linear.apply_quantized(q, s, M, y, residual=residual, path=native.PATH_GEMM_TILES)
        stop.record()
        torch.cuda.synchronize()
        seconds = start.elapsed_time(stop) / 1000 / launches
        tops = 2 * M * N * K / seconds / 1e12
        rows.append({"M": M, "K": K, "N": N, "residual": with_residual, "us": round(seconds * 1e6, 2),
                     "TOP/s": round(tops, 1), "frac": round(tops / INT8_PEAK_TOPS, 4)})
        del linear, x, q, s, y
    head = rows[0]
    return {"kernel": "gemm_kernel<true, Config<64, 2, 3, true>> (K <= 512; Config<128, 2, 2, true> above)", "bound": "mfma", "achieved": head["TOP/s"],
            "peak": INT8_PEAK_TOPS, "unit": "TOP/s", "frac": head["frac"], "traffic": None,
            "avg_launch_us": head["us"], "shape": {"M": head["M"], "K": head["K"], "N": head["N"]},
            "shapes": rows}


def qlinear_table(torch, native, rotate_bytes=1 << 30):
    """The isolated quantized linear: K=1024, N in {1024, 4096}, row scales
    U(0.001, 0.02) replicated over the K/256 blocks, int8 activations with
    fp32 block scales. For M in {1, 3, 64} every launch reads a different
    device copy of the weights, rotating through >= rotate_bytes of distinct
    matrices inside one captured HIP graph (more than the 256 MB MALL holds), so
    weights stream from HBM; per-launch time = graph time / launches, which
    includes each launch's own overhead. M in {1024, 4096} (MFMA-bound) run as
    plain launches on 4 rotating copies. bytes = K*N + 20*N (block scales, bias)
    + M*K + 16*M (int8 activations, scales) + 2*M*N (BF16 outputs)."""
    rng = np.random.default_rng(29)
    from tsac_hip.synthetic import random_linear

    K = 1024
    table = []
    for n in (1024, 4096):
        weights = random_linear(rng, K, n, row_scales=True)
        copies = max(4, -(-rotate_bytes // (K * n)))
        linears = [native.DeviceLinear(*weights) for _ in range(copies)]
        for m in (1, 3, 64, 1024, 4096):
            q = torch.randint(-127, 128, (m, K), dtype=torch.int8, device="cuda")
            s = torch.full((m, K // 256), 0.01, dtype=torch.float32, device="cuda")
            y = torch.empty((m, n), dtype=torch.int16, device="cuda")
            eager = torch.empty_like(y)
            linears[0].apply_quantized(q, s, m, eager)
            torch.cuda.synchronize()
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            if m <= 64:
                graph = torch.cuda.CUDAGraph()
                try:
                    # No weight copy may be freed while the graph is captured.
                    with torch.cuda.graph(graph, capture_error_mode="thread_local"):
                        for i in range(len(linears)):
                            linears[i].apply_quantized(q, s, m, y)
                except Exception as error:
                    raise RuntimeError(f"graph capture failed at N={n}, M={m}: {error}") from error
                launches, replays = len(linears), 3
                graph.replay()
                torch.cuda.synchronize()
                assert torch.equal(y, eager), "graph replay differs from the eager launch"
                start.record()
                for _ in range(replays):
                    graph.replay()
                stop.record()
                torch.cuda.synchronize()
                assert torch.equal(y, eager), "graph replay differs from the eager launch"
                seconds = start.elapsed_time(stop) / 1000 / (launches * replays)
                how = f"{launches} distinct {K * n >> 20} MiB weight copies rotated in one HIP graph"
                del graph
            else:
                reps = 20
                for i in range(4):
                    linears[i].apply_quantized(q, s, m, y)
                torch.cuda.synchronize()
                start.record()
                for i in range(reps):
                    linears[i % 4].apply_quantized(q, s, m, y)
                stop.record()
                torch.cuda.synchronize()
                assert torch.equal(y, eager)
                seconds = start.elapsed_time(stop) / 1000 / reps
                how = "plain launches over 4 rotating weight copies"
            traffic = K * n + 20 * n + m * K + 16 * m + 2 * m * n
            # The automatic path's choice: the small-M kernel also takes M <= 1024
            # when the GEMM's 128 x 128 tiles would fill at most a quarter of the CUs.
            units = torch.cuda.get_device_properties(0).multi_processor_count
            small = m <= 64 or (m <= 1024 and -(-m // 128) * -(-n // 128) * 4 <= units)
            table.append({"N": n, "M": m, "path": "gemv" if m <= 8 else "small-M MFMA" if small else "gemm",
                          "us": round(seconds * 1e6, 2),
                          "GB/s": round(traffic / seconds / 1e9, 1),
                          "frac_hbm": round(traffic / seconds / 1e9 / HBM_PEAK_GBPS, 4),
                          "TOP/s": round(2 * m * n * K / seconds / 1e12, 2), "method": how})
        del linears
        torch.cuda.empty_cache()
    return table


def attention_rates(torch, native, lengths=(256, 1290, 2580), batch=3, heads=16, head_width=64):
    """Causal attention alone (16 heads x 64, batch 3): full causal prefill
    (every query t over keys 0..t) and one incremental decode query over T
    cached keys, BF16 inputs drawn from N(0, 1), scale 1/8."""
    width = heads * head_width
    scale = 1.0 / np.sqrt(head_width)
    rows = []
    for T in lengths:
        gen = torch.Generator(device="cuda").manual_seed(T)
        qkv = (torch.randn((batch * T, 3 * width), device="cuda", generator=gen).view(torch.int32) >> 16)
        qkv = qkv.to(torch.int16).contiguous()
        start = torch.arange(batch, dtype=torch.int32, device="cuda") * T
        length = torch.full((batch,), T, dtype=torch.int32, device="cuda")
        replay = torch.zeros(batch, dtype=torch.int32, device="cuda")
        out = torch.empty((batch * T, width), dtype=torch.int16, device="cuda")
        run = lambda: native.attention_causal(qkv, heads, head_width, start, length, replay, batch, T, None,
                                              scale, out)
        run()
        start_e, stop_e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 10
        start_e.record()
        for _ in range(reps):
            run()
        stop_e.record()
        torch.cuda.synchronize()
        prefill_s = start_e.elapsed_time(stop_e) / 1000 / reps
        flops = batch * heads * 4 * head_width * T * (T + 1) / 2
        # Decode: the last position's query over the T cached keys/values,
        # rotating over copies of the caches that together exceed 1 GiB so
        # every launch reads its keys and values from HBM, not from cache.
        kv_bytes = batch * 2 * T * width * 2
        copies = -(-(1 << 30) // kv_bytes)
        keys = qkv[:, width:2 * width].contiguous().unsqueeze(0).repeat(copies, 1, 1)
        values = qkv[:, 2 * width:].contiguous().unsqueeze(0).repeat(copies, 1, 1)
        query = qkv.view(batch, T, 3 * width)[:, T - 1, :width].contiguous()
        dout = torch.empty((batch, width), dtype=torch.int16, device="cuda")
        # The C ABI called with pointers prepared up front, as a C caller would.
        lib, vp = native.library(), native.vp
        pointers = [(vp(keys[c].data_ptr()), vp(values[c].data_ptr())) for c in range(copies)]
        stream = vp(torch.cuda.current_stream().cuda_stream)
        q_pointer, out_pointer = vp(query.data_ptr()), vp(dout.data_ptr())

        def step(c):
            native.check(lib.tsac_hip_attention(q_pointer, *pointers[c], T * width, batch, T, heads, head_width,
                                                scale, 0, out_pointer, stream))
        for c in range(copies):
            step(c)
        reps = max(50, copies)
        torch.cuda.synchronize()
        start_e.record()
        for i in range(reps):
            step(i % copies)
        stop_e.record()
        torch.cuda.synchronize()
        decode_s = start_e.elapsed_time(stop_e) / 1000 / reps
        rows.append({"T": T, "prefill_us": round(prefill_s * 1e6, 1),
                     "prefill_TFLOPs": round(flops / prefill_s / 1e12, 2),
                     "prefill_frac_fp32_valu": round(flops / prefill_s / 1e12 / FP32_PEAK_TFLOPS, 4),
                     "decode_us": round(decode_s * 1e6, 2), "decode_cache_copies": copies,
                     "decode_GBps": round(kv_bytes / decode_s / 1e9, 1),
                     "decode_frac_hbm": round(kv_bytes / decode_s / 1e9 / HBM_PEAK_GBPS, 4)})
        del qkv, keys, values, out
    torch.cuda.empty_cache()
    return {"heads": heads, "head_width": head_width, "batch": batch, "rows": rows,
            "flops": "batch*heads*4*head_width*T*(T+1)/2 (causal prefill)",
            "bytes": "batch*2*T*heads*head_width*2 (decode: the BF16 key and value cache, rotated over "
                     "copies totalling over 1 GiB)"}


def frame_roofline(geometry, frames, batch, step_s):
    """The timed region's dominant kernel, up to 64 decode frame steps per
    launch: algorithmic bytes per step (every projection's int8 weights, block
    scales and bias read once per step for all lanes, plus each lane's
    temporal key/value cache rows at the average context position) over the
    average step time `step_s` (HIP events around the step loop on the
    session's stream / steps); per launch both scale by the launch's steps. It
    is bound by its ~240 dependent jobs on lane 0's chain, not by memory; the
    fraction shows how far from HBM-bound that is."""
    g = geometry
    record = "frame_step_decode_reference_2580frames.traffic.txt" if g.width == 512 else \
        "frame_step_decode_wide_2580frames.traffic.txt"
    measured, source = (recorded_traffic(record, "bytes_per_step") if frames == 2580 and batch == 3 else (None, None))

    def linear(k, n):
        return k * n + 4 * (k // 256) * n + 4 * n

    layer = (linear(g.width, 3 * g.width) + linear(g.width, g.width) + linear(g.width, g.ffn) +
             linear(g.ffn, g.width))
    lanes = min(batch, frames)
    steps = -(-frames // lanes)
    weights = (g.temporal_layers * layer + g.books * g.codebook_layers * layer + g.books * linear(g.width, g.alphabet)
               + (g.books - 1) * linear(g.latent, g.width) + linear(g.latent, g.width))
    cache = lanes * g.temporal_layers * ((steps - 1) / 2) * g.width * 2 * 2
    achieved = (weights + cache) / step_s / 1e9
    kernel = "frame_kernel<8, 32, 16, 128>" if g.width == 512 else "frame_kernel<16, 64, 16, 64>"
    return {"kernel": kernel, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured, "traffic_source": source,
            "limited_by": "dependent-job latency (~240 jobs per step in order on lane 0's chain)",
            "bytes_per_step": int(weights + cache), "avg_step_us": round(step_s * 1e6, 1), "steps": steps,
            "steps_per_launch": 64,
            "step_time": "GPU time between two HIP events around the frame-step loop on the session's stream, "
                         "divided by the steps"}


def round_trip(torch, native, geometry, frames, batch, steps, warmup, seed=1):
    """Encode + decode of frames x 12 codebooks (batch lanes, one group) on
    `geometry`, `steps` timed round trips after `warmup` untimed ones, bracketed
    by device synchronisations. Rate = tokens / (encode + decode seconds - the
    session-timed host-to-device copies of the calls' inputs)."""
    from tsac_hip.synthetic import random_model, random_tokens

    h = native.header(frames, batch, 1, 12)
    tokens = random_tokens(frames, 1, 12, seed=5)
    encode_s = decode_s = uploads = step_gpu = 0.0
    encode_split = [0.0, 0.0]
    decode_split = [0.0, 0.0]
    launches = set()
    # Every session and model is closed, and the device drained, before the
    # next part of the run (and before exit).
    with native.HipModel(random_model(geometry, seed=seed)) as hip_model, hip_model.session() as session:
        for _ in range(warmup):
            stream = session.encode(h, tokens)
            assert np.array_equal(session.decode(stream), tokens)
        torch.cuda.synchronize()
        # The C ABI takes host buffers (as MetalTransformer does); the session
        # times the host-to-device copy of each call's input separately, so the
        # reported rate is the one with inputs already in device memory.
        for _ in range(steps):
            t0 = time.perf_counter()
            stream = session.encode(h, tokens)
            t1 = time.perf_counter()
            e = session.timing()
            decoded = session.decode(stream)
            t2 = time.perf_counter()
            d = session.timing()
            encode_s += t1 - t0
            decode_s += t2 - t1
            encode_split[0] += e["model"]
            encode_split[1] += e["range_coding"]
            decode_split[0] += d["model"]
            decode_split[1] += d["range_coding"]
            uploads += e["input_upload"] + d["input_upload"]
            step_gpu += d["steps_gpu"] / d["steps"]
            launches.add(d["frame_launch"])
        torch.cuda.synchronize()
    assert np.array_equal(decoded, tokens), "round trip failed"
    encode_s /= steps
    decode_s /= steps
    uploads /= steps
    resident_s = encode_s + decode_s - uploads
    count = tokens.size
    return {
        "tokens_per_s": round(count / resident_s, 1),
        "ms_per_round_trip": round(1000 * resident_s, 2),
        "roofline": frame_roofline(geometry, frames, batch, step_gpu / steps),
        "pcie_inclusive_tokens_per_s": round(count / (encode_s + decode_s), 1),
        "input_upload_ms": round(1000 * uploads, 3),
        "encode_tokens_per_s": round(count / encode_s, 1),
        "decode_tokens_per_s": round(count / decode_s, 1),
        "token_stream_round_trip_s": round(encode_s + decode_s, 4),
        "stream_bytes": len(stream),
        "frame_launch": sorted(launches, key=str),
        "split_s": {"encode_model": round(encode_split[0] / steps, 4),
                    "encode_range_coding": round(encode_split[1] / steps, 4),
                    "decode_model": round(decode_split[0] / steps, 4),
                    "decode_range_coding": round(decode_split[1] / steps, 4),
                    "decode_frame_steps_gpu": round(step_gpu / steps * (-(-frames // batch)), 4)},
        "sample": f"encode + decode of {frames} frames x 12 codebooks, batch {batch}, {steps} timed round trips "
                  f"after {warmup} untimed",
        "geometry": {"width": geometry.width, "heads": geometry.heads, "head_width": geometry.head_width,
                     "ffn": geometry.ffn, "layers": [geometry.temporal_layers, geometry.codebook_layers]},
    }


def end_to_end(native, seconds, codebooks, batch, seed, steps=2):
    """AudioAnalyzer encode + decode of synthetic joint-stereo PCM on the GPU
    (DAC analysis, RVQ, probability model + range coding; then the model with
    the GPU range decoder, RVQ decoding, DAC synthesis), random-init DAC and
    reference-geometry transformer weights. Host wall clock around each call
    (PCM in and out of host memory included); the DAC-only passes are also timed
    alone to split the cost."""
    from tsac_hip.synthetic import REFERENCE, random_dac, random_model, synthetic_audio

    audio = synthetic_audio(seconds, 2, seed).astype(np.float32) / np.float32(32768)
    frames = -(-len(audio) // 512)
    padded = np.zeros((frames * 512, 2), np.float32)
    padded[:len(audio)] = audio
    with native.HipModel(random_model(REFERENCE, seed=1)) as hip_model, hip_model.session() as session, \
            native.HipDac(random_dac(2, 12, seed=1)) as dac:
        stream = dac.encode(session, audio, 2, codebooks=codebooks, entropy_batch=batch)
        pcm, _ = dac.decode(session, stream)
        encode_s = decode_s = 0.0
        for _ in range(steps):
            t0 = time.perf_counter()
            stream = dac.encode(session, audio, 2, codebooks=codebooks, entropy_batch=batch)
            t1 = time.perf_counter()
            pcm, channels = dac.decode(session, stream)
            t2 = time.perf_counter()
            encode_s += t1 - t0
            decode_s += t2 - t1
        assert channels == 2 and pcm.shape == (frames * 512, 2) and np.all(np.isfinite(pcm))
        t0 = time.perf_counter()
        tokens = dac.analyze(session, padded, frames, 1, codebooks)
        t1 = time.perf_counter()
        dac.synthesize(session, tokens, frames, 1, codebooks)
        t2 = time.perf_counter()
    encode_s /= steps
    decode_s /= steps
    return {"seconds_of_audio": seconds, "frames": frames, "codebooks": codebooks, "batch": batch,
            "encode_s": round(encode_s, 4), "decode_s": round(decode_s, 4),
            "round_trip_s": round(encode_s + decode_s, 4),
            "realtime_factor": round(seconds / (encode_s + decode_s), 1),
            "dac_analysis_rvq_s": round(t1 - t0, 4), "rvq_dac_synthesis_s": round(t2 - t1, 4),
            "stream_bytes": len(stream),
            "timing": "host wall clock around tsac_hip_audio_encode / tsac_hip_audio_decode, PCM in host memory"}


def cpu_end_to_end(seconds, codebooks, batch, seed):
    """The oracle's whole CPU chain (DAC analysis, RVQ, pack_normal; then
    unpack_normal, RVQ decoding, DAC synthesis) on `seconds` of the same
    synthetic audio, convolutions split over the host's cores, the model's
    lanes over at most `batch` threads."""
    sys.path.insert(0, str(ROOT / "oracle"))
    from oracle import Oracle, header
    from tsac_hip.synthetic import REFERENCE, random_dac, random_model, synthetic_audio

    cores = min(16, len(os.sched_getaffinity(0)))
    audio = synthetic_audio(seconds, 2, seed).astype(np.float32) / np.float32(32768)
    frames = -(-len(audio) // 512)
    padded = np.zeros((frames * 512, 2), np.float32)
    padded[:len(audio)] = audio
    o = Oracle()
    dm = o.dac_model(random_dac(2, 12, seed=1))
    om = o.model(random_model(REFERENCE, seed=1))
    threads = min(cores, batch)
    t0 = time.perf_counter()
    tokens = dm.analyze_audio(padded, frames, 1, threads=cores)
    t1 = time.perf_counter()
    h = header(frames, batch, 1, codebooks)
    selected = tokens.reshape(frames, 12)[:, :codebooks].copy()
    stream = om.pack_normal(h, selected, threads=threads)
    t2 = time.perf_counter()
    decoded = om.unpack_normal(stream, threads=threads)
    t3 = time.perf_counter()
    dm.synthesize_audio(tokens, frames, 1, threads=cores)
    t4 = time.perf_counter()
    assert np.array_equal(decoded, selected.ravel())
    return {"seconds": round(t4 - t0, 3), "analysis_s": round(t1 - t0, 3), "pack_normal_s": round(t2 - t1, 3),
            "unpack_normal_s": round(t3 - t2, 3), "synthesis_s": round(t4 - t3, 3), "cores": cores,
            "sample": f"{seconds} s of joint stereo ({frames} frames), {codebooks} codebooks, batch {batch}"}


def cpu_baseline(model, frames, batch):
    """The C oracle on a bounded sample of the same workload: a pack_normal +
    unpack_normal round trip of `frames` frames (same geometry, batch, books),
    lanes run concurrently like the reference's executor
    (src/common/transformer.cpp:70-90). Same rate definition as `value`:
    tokens / (encode seconds + decode seconds)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    from oracle import Oracle, header
    from tsac_hip.synthetic import random_tokens

    threads = min(len(os.sched_getaffinity(0)), batch)
    tokens = random_tokens(frames, 1, 12, seed=99)
    om = Oracle().model(model)
    t0 = time.perf_counter()
    stream = om.pack_normal(header(frames, batch, 1, 12), tokens, threads=threads)
    t1 = time.perf_counter()
    decoded = om.unpack_normal(stream, threads=threads)
    t2 = time.perf_counter()
    assert np.array_equal(decoded, tokens.ravel()), "oracle round trip failed"
    seconds = t2 - t0
    return {"value": round(tokens.size / seconds, 1), "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle pack_normal + unpack_normal round trip of {frames} frames x 12 codebooks "
                      f"(batch {batch}, {tokens.size} tokens, width {model.geometry.width}): encode {t1 - t0:.1f} s "
                      f"+ decode {t2 - t1:.1f} s; host has {len(os.sched_getaffinity(0))} cores, lane parallelism "
                      f"caps threads at {threads}; the rate is the one measured on this sample (a part of the "
                      f"2580-frame recording), not a time extrapolated to it"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the probability model runs on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    import torch

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    from tsac_hip import native
    from tsac_hip.synthetic import REFERENCE, WIDE, random_model

    geometry = REFERENCE if args.geometry == "reference" else WIDE
    result = {}
    if args.only in ("all", "model"):
        head = round_trip(torch, native, geometry, args.frames, args.batch, args.steps, args.warmup)
        result.update({"value": head.pop("tokens_per_s"), "ms_per_step": head.pop("ms_per_round_trip")})
        result.update(head)
    if args.only == "model":
        calibration_copy(torch)
    if args.only in ("all", "gemv", "gemm"):
        peaks = attainable_peaks(torch, native)
        result["attainable"] = peaks
    if args.only in ("all", "gemv"):
        roof = gemv_roofline(torch, native, args.gemv_launches)
        roof["frac_of_attainable"] = round(roof["achieved"] / peaks["hbm_read_GBps"], 4)
        result["roofline_gemv"] = roof
    if args.only in ("all", "gemm"):
        roof = gemm_roofline(torch, native)
        roof["frac_of_attainable"] = round(roof["achieved"] / peaks["int8_mfma_TOPs"], 4)
        result["roofline_gemm"] = roof
    if args.only in ("all", "attention"):
        result["attention"] = attention_rates(torch, native)
    if args.only in ("all", "reference") and args.geometry == "wide":
        result["reference_geometry"] = round_trip(torch, native, REFERENCE, 2580, 3, steps=3, warmup=1)
    if args.only in ("all", "qlinear"):
        result["qlinear"] = qlinear_table(torch, native)
    if args.only in ("all", "audio"):
        # The 30 s joint-stereo recording (12 codebooks, batch 3) and the 10 s
        # one (3 codebooks, automatic batch) end to end; the CPU chain on a
        # 1 s sample of the 30 s recording.
        audio = {"config4": end_to_end(native, 30.0, 12, 3, seed=4), "config0": end_to_end(native, 10.0, 3, 0, seed=3)}
        result["encode_decode_s_per_30s_stereo"] = audio["config4"]["round_trip_s"]
        if not args.no_cpu:
            cpu = cpu_end_to_end(1.0, 12, 3, seed=4)
            cpu["extrapolated_to_30s_s"] = round(cpu["seconds"] * 30.0, 1)
            cpu["extrapolation"] = "the 1 s sample's time x 30 (not measured on 30 s)"
            cpu["kind"] = "port"
            audio["cpu_baseline"] = cpu
            audio["config4_speedup_vs_cpu_extrapolated"] = round(
                cpu["extrapolated_to_30s_s"] / audio["config4"]["round_trip_s"], 1)
        result["end_to_end"] = audio
    if args.only == "all":
        if not args.no_cpu:
            frames = args.cpu_frames or (1290 if geometry is REFERENCE else 430)
            result["cpu_baseline"] = cpu_baseline(random_model(geometry, seed=1), frames, args.batch)
    line = {
        "metric": "prob-model tokens/s",
        "value": result.pop("value", None),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": result.pop("ms_per_step", None),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 (W8A8 int32-exact dots) + fp32/bf16",
        "data": "synthetic tokens, seeded random-init weights in the reference packed layout",
        "config": {"workload": f"encode+decode of a 30 s joint-stereo token stream: {args.frames} frames x "
                               f"12 codebooks, entropy batch {args.batch}, probability model of 12 + 3 layers, "
                               f"width {geometry.width}, {geometry.heads} x {geometry.head_width} heads, "
                               f"FFN {geometry.ffn}",
                   "frames": args.frames, "codebooks": 12, "batch": args.batch, "groups": 1,
                   "geometry": {"width": geometry.width, "heads": geometry.heads,
                                "head_width": geometry.head_width, "ffn": geometry.ffn,
                                "layers": [geometry.temporal_layers, geometry.codebook_layers]},
                   "parallelism": "single GPU"},
        "baseline_metrics": "prob-model tokens/s; qlinear HBM GB/s; encode+decode s per 30 s stereo",
    }
    line.update(result)
    print(json.dumps(line), flush=True)
    torch.cuda.synchronize()


if __name__ == "__main__":
    main()
