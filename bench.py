"""Benchmark of the hot path: quantized decode GEMV on one MI355X.

Workload (the shape the metric is quoted on):
Q4_K output-rows weight, K=4096, N=14336, M=1 f32 activation row, F32 mode.
Inputs are resident in HBM before the timed region. The weight is held in C
copies (C x 33 MB >= 512 MB, above the 256 MB Infinity Cache) and a step is
one GEMV over each copy in turn (C launches, back to back), so every launch
streams its weight from HBM and the event region's fixed cost is spread over
C x steps launches; the region's own cost (events with no launch between
them) is measured and reported beside it.

Prints ONE JSON line (the driver's contract) with a `roofline` object for the
GEMV kernel (algorithmic bytes per launch / the average launch duration from
HIP events on the launch stream, vs 8 TB/s) and a `cpu_baseline` object (the
oracle's CpuScalar port on one host core). The line also carries:
- `gemv_q8_0`: the same measurement for Q8_0 at 4096 x 14336 (the north
  star's GEMV target names Q4_K and Q8_0);
- `gemm`: the prefill GEMM at M=2048, K=4096, N=12288 for Q4_K and Q8_0,
  TFLOP/s against the dense f16 matrix-core peak (the north star's GEMM
  target);
- `e2e`: Qwen3-8B-shape decode tokens/s of the GPU-resident decoder
  with its own roofline and CPU baseline, and
  whether its greedy ids equal the CPU run's (tests/golden/qwen3_8b_greedy.json).

Inputs are synthetic, drawn by the library's own host functions: N(0, 0.02^2)
weights (configs[2] and [3]: 0.5% N(0, 0.2^2) outliers for the K-quants) from
qi_hip_synth_normal, quantized by qi_hip_quantize (the reference quantizer,
f16 storage rounding), activations N(0, 1). The e2e model is the recipe of
quantinfer_amd.synth. Nothing in the measured legs touches the test oracle;
it is loaded only for the cpu_baseline legs.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
K, N, M = 4096, 14336, 1
WIRE = {1: 34, 2: 18, 3: 144, 4: 176, 5: 210}
BLOCK = {1: 32, 2: 32, 3: 256, 4: 256, 5: 256}
QNAME = {1: "q8_0", 2: "q4_0", 3: "q4_k", 4: "q5_k", 5: "q6_k"}


def algorithmic_bytes(qtype: int, k: int, n: int, m: int) -> int:
    """GGUF wire weight bytes + activations + outputs (f32)."""
    return n * (k // BLOCK[qtype]) * WIRE[qtype] + m * k * 4 + m * n * 4


def traffic_from_profile(name: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.]+)", open(path).read())
    return float(m.group(1)) if m else None


def weight_blocks(qtype: int, k: int, n: int, seed: int):
    """Output-rows blocks of an f32 [N, K] weight drawn from N(0, 0.02^2), with
    0.5% N(0, 0.2^2) outliers for the K-quants,
    quantized by the reference quantizer with f16 storage rounding
    (qi_hip_synth_normal, qi_hip_quantize)."""
    import quantinfer_amd as qa
    outliers = 0.005 if qtype >= 3 else 0.0
    w = qa.synth_normal(seed, n * k, 0.02, outliers, 0.2)
    return qa.quantize(qtype, w, storage_f16=True)


def normal(seed: int, n: int, std: float = 1.0):
    import quantinfer_amd as qa
    return qa.synth_normal(seed, n, std)


def gemv_bench(qtype: int, k: int, n: int, m: int, steps: int, warmup: int, copies_mb: float = 512.0,
               with_abi: bool = False, row_major: bool = False) -> dict:
    """`steps` passes over C resident weight copies, one launch per copy,
    event-timed on the launch stream; plus the event region's own cost.
    row_major: the weight in the QuantInfer layout (K rows of N / bs blocks
    along N, backends/cpu/src/matmul.rs:14-90)."""
    import quantinfer_amd as qa
    from quantinfer_amd import hiprt

    ctx = qa.Context(0)
    blocks = weight_blocks(qtype, n, k, seed=0x5EED0000 + qtype) if row_major else \
        weight_blocks(qtype, k, n, seed=0x5EED0000 + qtype)
    wbytes = n * (k // BLOCK[qtype]) * WIRE[qtype]
    copies = max(1, int(-(-copies_mb * 1e6 // wbytes)))
    layout = qa.ROW_MAJOR if row_major else qa.OUTPUT_ROWS
    weights = [ctx.weights(qtype, layout, k, n, blocks) for _ in range(copies)]
    x = hiprt.DeviceBuffer.from_array(normal(0x5EED1000, m * k).reshape(m, k))
    y = hiprt.DeviceBuffer(m * n * 4)
    stream = hiprt.Stream()

    def step():
        for w in weights:
            w.linear_device(x.ptr, m, y.ptr, qa.MODE_F32, stream.handle)

    for _ in range(warmup):
        step()
    stream.synchronize()
    start, end = hiprt.Event(), hiprt.Event()
    # the event region's fixed cost: the two events with nothing between them
    empty = []
    for _ in range(5):
        start.record(stream)
        end.record(stream)
        stream.synchronize()
        empty.append(start.elapsed_ms(end))
    # timed region: `steps` passes over the copies, bracketed by HIP events on
    # the stream the kernels are launched on
    hiprt.synchronize()
    start.record(stream)
    for _ in range(steps):
        step()
    end.record(stream)
    stream.synchronize()
    region_ms = start.elapsed_ms(end)
    out = {"region_ms": region_ms, "copies": copies, "launches": steps * copies,
           "empty_region_us": statistics.median(empty) * 1e3, "device": ctx.device_name()}

    if with_abi:
        # PCIe-inclusive rate, never `value`: the synchronous KernelBackend
        # call (qi_hip_linear: host x in, host y out), timed on the host
        xh = normal(0x5EED1000, m * k).reshape(m, k)
        abi_times = []
        for i in range(100):
            t = time.perf_counter()
            weights[i % copies].linear(xh, qa.MODE_F32)
            abi_times.append(time.perf_counter() - t)
        out["abi_ms"] = statistics.median(abi_times) * 1e3
        out["abi_calls"] = len(abi_times)
    start.destroy()
    end.destroy()
    for w in weights:
        w.free()
    x.free()
    y.free()
    stream.destroy()
    ctx.close()
    return out


def gemv_line(qtype: int, k: int, n: int, m: int, g: dict, steps: int, warmup: int,
              row_major: bool = False) -> dict:
    """The JSON object of one GEMV measurement."""
    abytes = algorithmic_bytes(qtype, k, n, m)
    us_launch = g["region_ms"] * 1e3 / g["launches"]
    gbps = abytes / (us_launch * 1e-6) / 1e9
    q = QNAME[qtype]
    lay = "row_major" if row_major else "output_rows"
    return {
        "metric": f"quant GEMV GB/s (% of HBM peak) at {k}x{n}",
        "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(g["region_ms"] / steps, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": f"synthetic: N(0,0.02^2) weights{' with 0.5% N(0,0.2^2) outliers' if qtype >= 3 else ''}"
                f" quantized to {q} (qi_hip_quantize, f16 storage); x ~ N(0,1)",
        "config": {"workload": f"{q}_gemv_{lay}_m{m}_k{k}_n{n}", "qtype": q, "m": m, "k": k,
                   "n": n, "mode": "f32", "weight_copies": g["copies"],
                   "step": f"one GEMV launch over each of the {g['copies']} resident weight copies",
                   "launches": g["launches"], "us_per_launch": round(us_launch, 3),
                   "event_region_overhead_us": round(g["empty_region_us"], 2), "device": g["device"]},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": traffic_from_profile(f"{q}_gemv_row_major_{k}x{n}_traffic.md" if row_major
                                                     else f"{q}_gemv_{k}x{n}_traffic.md" if m == 1
                                                     else f"{q}_gemv_m{m}_{k}x{n}_counters.md")},
    }


def copy_calibration(steps: int, mib: int = 256) -> None:
    """`steps` device-to-device copies of `mib` MiB (the HIP runtime's copy
    kernel): the known-size reference that scales rocprofv3's FETCH_SIZE and
    WRITE_SIZE readings into bytes."""
    from quantinfer_amd import hiprt

    nbytes = mib << 20
    src, dst = hiprt.DeviceBuffer(nbytes), hiprt.DeviceBuffer(nbytes)
    stream = hiprt.Stream()
    dst.copy_from(src, nbytes, stream)
    stream.synchronize()
    start, end = hiprt.Event(), hiprt.Event()
    start.record(stream)
    for _ in range(steps):
        dst.copy_from(src, nbytes, stream)
    end.record(stream)
    stream.synchronize()
    us = start.elapsed_ms(end) * 1e3 / steps
    print(json.dumps({"calibration": "d2d_copy", "bytes_read_per_copy": nbytes,
                      "bytes_written_per_copy": nbytes, "copies": steps, "us_per_copy": round(us, 2)}))
    for b in (src, dst):
        b.free()
    stream.destroy()


MFMA_F16_PEAK_TFLOPS = 2500.0

# Sizes of the streaming-read calibration: the decode GEMV weights at the
# Qwen3-8B projection shapes (Q4_K 4096x4096, 4096x6144, 12288x4096,
# 4096x14336, 4096x24576; Q8_0 4096x14336), then 512 MB and 1 GiB.
CALIB_BYTES = [9437184, 14155776, 28311552, 33030144, 56623104, 62390272, 509607936, 1073741824]


def calib_bench(steps: int = 10) -> dict:
    """Plain streaming reads (quantinfer_amd/calib, not the product library)
    at the GEMV weight sizes, timed as gemv_bench times the GEMV: back to
    back over resident zero-filled buffers (at least 512 MB in all), HIP
    events on the launch stream, best of three regions. The ceiling a kernel
    that reads each byte once reaches at that size with this launch pattern."""
    import ctypes

    from quantinfer_amd import build as qb, hiprt

    if not os.path.exists(qb.CALIB_LIB):
        raise RuntimeError(f"{qb.CALIB_LIB} is not built (python quantinfer_amd/build.py)")
    cal = ctypes.CDLL(qb.CALIB_LIB)
    cal.qi_calib_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int32, ctypes.c_uint64,
                                         ctypes.c_void_p, ctypes.c_void_p]
    sink = hiprt.DeviceBuffer(4096)
    stream = hiprt.Stream()
    patterns = [("grid-stride", 0, w) for w in (512, 1024, 2048, 4096)] + \
               [("chunk", 1, c) for c in (36864, 73728)]
    rows = []
    for nbytes in CALIB_BYTES:
        copies = max(1, -(-512_000_000 // nbytes))
        bufs = [hiprt.DeviceBuffer(nbytes) for _ in range(copies)]
        for b in bufs:
            b.zero()
        for name, pat, param in patterns:
            def step():
                for b in bufs:
                    err = cal.qi_calib_stream_read(b.ptr, nbytes, pat, param, sink.ptr, stream.handle)
                    if err:
                        raise RuntimeError(f"qi_calib_stream_read: HIP error {err}")
            for _ in range(3):
                step()
            stream.synchronize()
            n = max(steps, -(-2_000_000_000 // (nbytes * copies)))
            best = None
            for _ in range(3):
                a, b = hiprt.Event(), hiprt.Event()
                a.record(stream)
                for _ in range(n):
                    step()
                b.record(stream)
                us = a.elapsed_ms(b) * 1e3 / (n * copies)
                best = us if best is None else min(best, us)
                a.destroy()
                b.destroy()
            rows.append({"bytes": nbytes, "pattern": name,
                         "param": f"{param} workgroups" if pat == 0 else f"{param} B per workgroup",
                         "us_per_read": round(best, 3), "gb_s": round(nbytes / best / 1e3, 1)})
        for b in bufs:
            b.free()
    sink.free()
    stream.destroy()
    best = {}
    for r in rows:
        if r["bytes"] not in best or r["gb_s"] > best[r["bytes"]]["gb_s"]:
            best[r["bytes"]] = r
    return {"calibration": "streaming_read", "unit": "GB/s", "peak": HBM_PEAK_GBPS,
            "note": "plain non-temporal 16-byte loads, event-timed back to back like the GEMV; "
                    "best pattern per size below, every pattern in `rows`",
            "best": [{"bytes": b, "gb_s": r["gb_s"], "frac": round(r["gb_s"] / HBM_PEAK_GBPS, 4),
                      "us_per_read": r["us_per_read"], "pattern": f"{r['pattern']} ({r['param']})"}
                     for b, r in sorted(best.items())],
            "rows": rows}


def timeline_bench(qtype: int, k: int, n: int, m: int = 1) -> dict:
    """Workgroup timeline of the decode GEMV kernel from the profiling build
    (libqi_hip_timeline.so, python quantinfer_amd/build.py --timeline): the
    launch stream runs passes over resident weight copies as gemv_bench does;
    the stamps of the last launch are read back. Times are microseconds from
    the first workgroup's start (100 MHz clock), as percentiles over
    workgroups. With two or more rows the stamps cover the GEMV kernel
    between the activation-record and split-K-sum kernels; "activations in
    LDS" is then the records' copy into LDS."""
    import ctypes

    import numpy as np

    import quantinfer_amd as qa
    from quantinfer_amd import build as qb, hiprt

    if not os.path.exists(qb.TIMELINE_LIB):
        raise RuntimeError(f"{qb.TIMELINE_LIB} is not built (python quantinfer_amd/build.py --timeline)")
    qa.LIB_PATH = qb.TIMELINE_LIB
    lib = qa.lib()
    lib.qi_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
    ctx = qa.Context(0)
    blocks = weight_blocks(qtype, k, n, seed=0x5EED0000 + qtype)
    wbytes = n * (k // BLOCK[qtype]) * WIRE[qtype]
    copies = max(2, -(-512_000_000 // wbytes))
    weights = [ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks) for _ in range(copies)]
    x = hiprt.DeviceBuffer.from_array(normal(0x5EED1000, m * k).reshape(m, k))
    y = hiprt.DeviceBuffer(m * n * 4)
    stream = hiprt.Stream()
    for _ in range(4):
        for w in weights:
            w.linear_device(x.ptr, m, y.ptr, qa.MODE_F32, stream.handle)
    stream.synchronize()
    if lib.qi_timeline_clear() != 0:
        raise RuntimeError("qi_timeline_clear failed")
    for w in weights:
        w.linear_device(x.ptr, m, y.ptr, qa.MODE_F32, stream.handle)
    stream.synchronize()
    ts = np.zeros(8192 * 8, dtype=np.uint64)
    if lib.qi_timeline_read(ts.ctypes.data, ts.size) != 0:
        raise RuntimeError("qi_timeline_read failed")
    ts = ts.reshape(8192, 8)
    used = ts[:, 0] > 0
    t = ts[used].astype(np.int64)
    rel = (t[:, :5] - t[:, 0].min()) / 100.0  # 100 MHz ticks -> us
    # HW_ID bits 8-11 CU, 12 shader array, 13-15 shader engine; plus the XCD
    cus = {(int(r[6]), int(r[5]) >> 8 & 0xFF) for r in ts[used]}
    pct = (0, 10, 50, 90, 100)

    def dist(v):
        return {f"p{p}": round(float(np.percentile(v, p)), 3) for p in pct}

    for w in weights:
        w.free()
    x.free()
    y.free()
    stream.destroy()
    ctx.close()
    return {
        "timeline": f"{QNAME[qtype]}_gemv_output_rows_m{m}_k{k}_n{n}", "workgroups": int(used.sum()),
        "compute_units": len(cus), "weight_bytes": wbytes, "unit": "us from the first workgroup's start",
        "start": dist(rel[:, 0]), "records_in_lds": dist(rel[:, 1]), "first_batch_done": dist(rel[:, 2]),
        "units_done": dist(rel[:, 3]), "epilogue": dist(rel[:, 4]),
        "prep_wait": dist(rel[:, 1] - rel[:, 0]), "after_prep_to_first_batch": dist(rel[:, 2] - rel[:, 1]),
    }


def library_f16_gemm(m: int, k: int, n: int, steps: int = 20) -> dict:
    """The same GEMM shape as a plain f16 library GEMM (torch.matmul, which
    calls hipBLASLt), operands resident, no dequantization: what a vendor
    GEMM reaches at this shape on this box, for scale. Its own process
    (--workload libgemm): torch bundles its own HIP runtime, and the second
    runtime to start in a process finds no device."""
    import torch

    x = torch.randn(m, k, device="cuda", dtype=torch.float16)
    w = torch.randn(n, k, device="cuda", dtype=torch.float16) * 0.02
    for _ in range(5):
        x @ w.t()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        x @ w.t()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    del x, w
    torch.cuda.empty_cache()
    return {"what": "torch.matmul f16 (hipBLASLt), x[m,k] @ w[n,k]^T", "value": round(tflops, 1),
            "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "ms": round(ms, 5)}


def gemm_bench(qtype: int, m: int, k: int, n: int, steps: int, warmup: int, mode: str = "mfma") -> dict:
    """Prefill GEMM: `steps` back-to-back linear calls on resident inputs (two
    weight copies alternating), event-timed on the launch stream. mode "mfma":
    the f16-operand GEMM (each call the f16 activation conversion plus the
    GEMM); mode "f32": F32 mode, which for Q4_K / Q5_K from 48 rows is the
    split-half GEMM (each call the activation halves plus the GEMM, and the
    split-K sum where the shape takes one), within the f32 GEMV's bars."""
    import quantinfer_amd as qa
    from quantinfer_amd import hiprt

    qmode = {"mfma": qa.MODE_MFMA, "f32": qa.MODE_F32}[mode]

    ctx = qa.Context(0)
    blocks = weight_blocks(qtype, k, n, seed=0x5EED0010 + qtype)
    weights = [ctx.weights(qtype, qa.OUTPUT_ROWS, k, n, blocks) for _ in range(2)]
    x = hiprt.DeviceBuffer.from_array(normal(0x5EED3000, m * k).reshape(m, k))
    y = hiprt.DeviceBuffer(m * n * 4)
    stream = hiprt.Stream()
    for i in range(warmup):
        weights[i % 2].linear_device(x.ptr, m, y.ptr, qmode, stream.handle)
    stream.synchronize()
    start, end = hiprt.Event(), hiprt.Event()
    start.record(stream)
    for i in range(steps):
        weights[i % 2].linear_device(x.ptr, m, y.ptr, qmode, stream.handle)
    end.record(stream)
    stream.synchronize()
    ms = start.elapsed_ms(end) / steps
    name = ctx.device_name()
    for w in weights:
        w.free()
    for b in (x, y):
        b.free()
    stream.destroy()
    ctx.close()
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    qname = QNAME[qtype]
    f32 = mode == "f32"
    return {
        "metric": "prefill GEMM TFLOP/s (% of dense f16 MFMA peak)",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": ("f32 activations as two f16 halves x exact f16 codes, f32 accumulation" if f32
                  else "f16 operands, f32 accumulation"),
        "data": f"synthetic: N(0,0.02^2) weights{' with 0.5% outliers' if qtype >= 3 else ''} quantized "
                f"to {qname} (qi_hip_quantize); x ~ N(0,1)",
        "config": {"workload": f"{qname}_gemm_output_rows_m{m}_k{k}_n{n}", "qtype": qname,
                   "m": m, "k": k, "n": n, "mode": mode,
                   "step": ("one linear call: activation halves + split-half GEMM" if f32
                            else "one linear call: f16 activation conversion + GEMM"), "device": name},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": None},
        **({"note": "two f16 matrix instructions per product (the activation halves): the useful "
                    "rate is bounded by half the dense f16 peak"} if f32 else {}),
    }


MFMA_F32_PEAK_TFLOPS = 157.3


def f32_head_bench(steps: int, warmup: int) -> dict:
    """F32 weights through the dense `matmul` (backends/cpu/src/backend.rs:48-60):
    the unchanged runtime's LM head, [4096, 151936] f32 (a Q6_K head is
    dequantized at load, runtime/src/qwen3/loader.rs:47-61). One decode row
    (the streaming F32 GEMV, HBM-bound on 2.49 GB), the 512-row prompt's
    logits (the f32 matrix-core GEMM, f32w_gemm_kernel, against the f32
    matrix-core peak), and the
    synchronous per-token call with host buffers as the runtime makes it."""
    import quantinfer_amd as qa
    from quantinfer_amd import hiprt

    k, n = 4096, 151936
    ctx = qa.Context(0)
    w = ctx.weights(qa.F32, qa.ROW_MAJOR, k, n, normal(0x5EED9000, k * n, 0.02))
    stream = hiprt.Stream()
    out = {}
    for m in (1, 512):
        x = hiprt.DeviceBuffer.from_array(normal(0x5EED9001, m * k).reshape(m, k))
        y = hiprt.DeviceBuffer(m * n * 4)
        reps = steps if m == 1 else max(steps // 4, 5)
        for _ in range(warmup):
            w.linear_device(x.ptr, m, y.ptr, qa.MODE_AUTO, stream.handle)
        stream.synchronize()
        start, end = hiprt.Event(), hiprt.Event()
        start.record(stream)
        for _ in range(reps):
            w.linear_device(x.ptr, m, y.ptr, qa.MODE_AUTO, stream.handle)
        end.record(stream)
        stream.synchronize()
        out[m] = start.elapsed_ms(end) / reps
        x.free()
        y.free()
    xh = normal(0x5EED9001, k).reshape(1, k)
    times = []
    for _ in range(20):
        t = time.perf_counter()
        w.linear(xh, qa.MODE_AUTO)
        times.append(time.perf_counter() - t)
    abi_ms = statistics.median(times) * 1e3
    stream.destroy()
    w.free()
    ctx.close()
    gemv_bytes = k * n * 4 + k * 4 + n * 4
    gbps = gemv_bytes / (out[1] * 1e-3) / 1e9
    tflops = 2.0 * 512 * k * n / (out[512] * 1e-3) / 1e12
    return {
        "metric": "F32 matmul (unchanged runtime's LM head) GB/s at M=1",
        "value": round(gbps, 2), "unit": "GB/s", "dtype": "f32",
        "config": {"workload": "f32_matmul_row_major_k4096_n151936", "k": k, "n": n, "mode": "auto"},
        "m1_ms": round(out[1], 4),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None},
        "m512": {"ms": round(out[512], 3), "tflops": round(tflops, 2), "kernel": "f32w_gemm_kernel (v_mfma_f32_16x16x4f32)",
                 "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_F32_PEAK_TFLOPS,
                              "unit": "TFLOP/s", "frac": round(tflops / MFMA_F32_PEAK_TFLOPS, 4)}},
        "through_abi_m1_ms": round(abi_ms, 4),
        "note": "through_abi: qi_hip_linear with host x and y (H2D 16 KB, GEMV, D2H 608 KB), the "
                "per-token cost of the head when the unchanged runtime calls KernelBackend::matmul",
    }


def host_cpu() -> str:
    """The host CPU model and the logical CPU count this process may use."""
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 0
    return f"{model} ({avail} CPUs available)"


def cpu_baseline(qtype: int, repeats: int = 3):
    """The oracle's port of CpuScalar::matmul_q4_k_output_rows (single-threaded,
    as the reference's output-row kernels are), pinned to one host core."""
    from oracle import pyoracle as po

    blocks = weight_blocks(qtype, K, N, seed=0x5EED0000 + qtype)
    x = normal(0x5EED1000, M * K).reshape(M, K)
    try:
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {min(old)})
    except (AttributeError, OSError):
        old = None
    times = []
    try:
        for _ in range(repeats):
            t = time.perf_counter()
            po.matmul_output_rows(qtype, x, blocks, N)
            times.append(time.perf_counter() - t)
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    sec = statistics.median(times)
    return {
        "value": round(algorithmic_bytes(qtype, K, N, M) / sec / 1e9, 3),
        "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"full workload (M=1, K={K}, N={N}) x{repeats}, median {sec * 1e3:.1f} ms; "
                  f"oracle C port of CpuScalar output-row kernel, 1 pinned core of "
                  f"{host_cpu()}; Q4_K has no cpu-simd path in the reference",
    }


def cpu_simd_table(repeats: int = 3) -> dict:
    """The reference's two CPU kernels for Q8_0/Q4_0 output rows, one pinned
    core each: the scalar CpuScalar order (matmul.rs:119-160) and the cpu-simd
    per-block dot (cpu-simd lib.rs:179-204; AVX-512 where the host has it, else
    AVX2), on BASELINE configs[0] (Q8_0, K = N = 4096) and a configs[1] shape
    (Q4_0, K = 4096, N = 12288), M = 1. GB/s of algorithmic bytes."""
    from oracle import pyoracle as po

    isa = 2 if po.simd_available(2) else (1 if po.simd_available(1) else 0)
    rows = []
    try:
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {min(old)})
    except (AttributeError, OSError):
        old = None
    try:
        for qtype, name, k, n in ((1, "q8_0", 4096, 4096), (2, "q4_0", 4096, 12288)):
            blocks = weight_blocks(qtype, k, n, seed=0x5EED0000 + qtype)
            x = normal(0x5EED1000, k).reshape(1, k)
            row = {"qtype": name, "k": k, "n": n, "m": 1}
            legs = [("scalar", lambda: po.matmul_output_rows(qtype, x, blocks, n))]
            if isa:
                legs.append(("simd", lambda: po.matmul_output_rows_simd(qtype, isa, x, blocks, n)))
            for leg, fn in legs:
                times = []
                for _ in range(repeats):
                    t = time.perf_counter()
                    fn()
                    times.append(time.perf_counter() - t)
                sec = statistics.median(times)
                row[leg + "_ms"] = round(sec * 1e3, 3)
                row[leg + "_gbps"] = round(algorithmic_bytes(qtype, k, n, 1) / sec / 1e9, 3)
            rows.append(row)
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    return {"cpu_simd_table": rows, "isa": {0: "none", 1: "avx2", 2: "avx512f"}[isa], "cores": 1,
            "host": host_cpu(), "kind": "port"}


# ------------------------------------------------ every BASELINE config point

# (BASELINE.json configs index, qtype, K, N, row counts) of the decode GEMV
# points: configs[0] Q8_0 4096^2; configs[1] Q4_0 at the four Qwen3-8B
# projection shapes; configs[2] Q4_K / Q5_K / Q6_K in both FFN orientations.
GEMV_POINTS = ([(0, 1, 4096, 4096, (1,))] +
               [(1, 2, k, n, (1, 4, 16)) for k, n in ((4096, 4096), (4096, 1024), (4096, 12288), (12288, 4096))] +
               [(2, q, k, n, (1, 8)) for q in (3, 4, 5) for k, n in ((4096, 14336), (14336, 4096))])
# The same points on row-major weights (QuantInfer layout, blocks along N:
# backends/cpu/src/matmul.rs:14-90), the tiled row-major image: Q4_K at the
# FFN up shape, Q4_0 at 4096 x 12288, Q8_0 at 4096^2, at their configs' row
# counts (one row on the row-major GEMV, from 3 rows the row-major GEMM).
RM_POINTS = [(2, 3, 4096, 14336, (1, 8)), (1, 2, 4096, 12288, (1, 4, 16)), (0, 1, 4096, 4096, (1,))]
# the prefill GEMM, Q8_0 and Q4_K, M x (K, N)
GEMM_POINTS = [(3, q, k, n, (128, 512, 2048)) for q in (1, 3)
               for k, n in ((4096, 4096), (4096, 12288), (12288, 4096))]
RIDGE_FLOP_PER_BYTE = MFMA_F16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBPS * 1e9)


class _OneCore:
    """Pin this process to one host core for the CPU legs (the reference's
    output-row kernels are single-threaded, backends/cpu/src/config.rs:59-67)."""

    def __enter__(self):
        try:
            self.old = os.sched_getaffinity(0)
            os.sched_setaffinity(0, {min(self.old)})
        except (AttributeError, OSError):
            self.old = None
        return self

    def __exit__(self, *exc):
        if self.old is not None:
            os.sched_setaffinity(0, self.old)


def _median_s(fn, repeats: int) -> float:
    times = []
    for _ in range(repeats):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return statistics.median(times)


def _cpu_point(qtype: int, k: int, n: int, m: int, blocks, unit: str, work: float,
               row_major: bool = False) -> dict:
    """CpuScalar (and, for Q8_0/Q4_0 output rows, the cpu-simd per-block
    dot, cpu-simd lib.rs:179-204) on one pinned core over `rows` <= m
    activation rows, scaled linearly to m rows (rows are independent,
    matmul.rs:146-158). `work` is the point's bytes (GB/s) or flops
    (TFLOP/s). row_major: CpuScalar's blocks-along-N matmul (matmul.rs:14-90)."""
    from oracle import pyoracle as po

    rows = m if m <= 4 else 2
    x = normal(0x5EED8100 + m, rows * k).reshape(rows, k)
    isa = 2 if po.simd_available(2) else (1 if po.simd_available(1) else 0)
    if row_major:
        legs = [("scalar", lambda: po.matmul_row_major(qtype, x, blocks, n))]
    else:
        legs = [("scalar", lambda: po.matmul_output_rows(qtype, x, blocks, n))]
    if qtype in (1, 2) and isa and not row_major:
        legs.append(("simd", lambda: po.matmul_output_rows_simd(qtype, isa, x, blocks, n)))
    out = {"unit": unit, "cores": 1, "kind": "port"}
    with _OneCore():
        for leg, fn in legs:
            sec = _median_s(fn, 3 if rows * k * n <= 64 << 20 else 1) * m / rows
            out[leg] = round(work / sec / (1e9 if unit == "GB/s" else 1e12), 6 if unit == "TFLOP/s" else 3)
            out[leg + "_ms"] = round(sec * 1e3, 2)
    if "simd" not in out:
        out["simd"] = None
    out["value"] = out["scalar"]
    out["sample"] = (f"{rows} of {m} rows, scaled x{m // rows}" if rows < m else f"all {m} rows") + \
        (f"; oracle C port of CpuScalar's row-major matmul (matmul.rs:14-90)" if row_major else
         f"; oracle C port of CpuScalar (matmul.rs:119-160, :282-332)") + \
        (f" and the cpu-simd {['', 'avx2', 'avx512f'][isa]} block dot" if len(legs) > 1 else
         ("; no cpu-simd path for K-quants in the reference" if qtype >= 3 else "")) + \
        f"; 1 pinned core of {host_cpu()}"
    return out


def _time_rotating(weights, m: int, k: int, n: int, mode: int, steps: int, warmup: int) -> float:
    """Microseconds per linear_device call, rotating over resident weight
    copies, HIP events on the launch stream."""
    import quantinfer_amd as qa
    from quantinfer_amd import hiprt

    x = hiprt.DeviceBuffer.from_array(normal(0x5EED1000, m * k).reshape(m, k))
    y = hiprt.DeviceBuffer(m * n * 4)
    stream = hiprt.Stream()
    calls = 0
    for _ in range(warmup):
        for w in weights:
            w.linear_device(x.ptr, m, y.ptr, mode, stream.handle)
    stream.synchronize()
    start, end = hiprt.Event(), hiprt.Event()
    start.record(stream)
    for _ in range(steps):
        for w in weights:
            w.linear_device(x.ptr, m, y.ptr, mode, stream.handle)
            calls += 1
    end.record(stream)
    stream.synchronize()
    us = start.elapsed_ms(end) * 1e3 / calls
    for b in (start, end):
        b.destroy()
    x.free()
    y.free()
    stream.destroy()
    return us


def configs_table(steps: int, warmup: int, with_cpu: bool) -> dict:
    """Every BASELINE.json config point of the linear path, each with its
    time per call, its rate against its roofline and (unless with_cpu is
    false) the CPU kernels beside it. GEMV points: F32 mode, one call per
    resident weight copy (copies >= 512 MB), GB/s of algorithmic bytes
    against 8 TB/s. GEMM points: MFMA mode (f16 operands, f32 accumulation),
    TFLOP/s against the attainable roofline min(2.5 PFLOP/s, intensity x
    8 TB/s), and beside it F32 mode (the split-half GEMM); weight copies
    rotated the same way."""
    import quantinfer_amd as qa

    ctx = qa.Context(0)
    out = {"gemv": [], "gemv_row_major": [], "gemm": []}
    for kind, points in (("gemv", GEMV_POINTS), ("gemv_row_major", RM_POINTS), ("gemm", GEMM_POINTS)):
        for cfg_i, qtype, k, n, ms in points:
            row_major = kind == "gemv_row_major"
            # row major: K rows of N / bs blocks along N
            blocks = weight_blocks(qtype, n, k, seed=0x5EED0000 + qtype) if row_major else \
                weight_blocks(qtype, k, n, seed=0x5EED0000 + qtype)
            wbytes = n * (k // BLOCK[qtype]) * WIRE[qtype]
            copies = max(2, int(-(-512e6 // wbytes)))
            layout = qa.ROW_MAJOR if row_major else qa.OUTPUT_ROWS
            weights = [ctx.weights(qtype, layout, k, n, blocks) for _ in range(copies)]
            for m in ms:
                abytes = algorithmic_bytes(qtype, k, n, m)
                if kind != "gemm":
                    us = _time_rotating(weights, m, k, n, qa.MODE_F32, steps, warmup)
                    gbps = abytes / (us * 1e-6) / 1e9
                    entry = {"config": cfg_i, "qtype": QNAME[qtype], "m": m, "k": k, "n": n,
                             "us": round(us, 3), "gbps": round(gbps, 1),
                             "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                                          "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                                          "algorithmic_bytes": abytes}}
                    if with_cpu:
                        entry["cpu_baseline"] = _cpu_point(qtype, k, n, m, blocks, "GB/s", abytes, row_major)
                else:
                    reps = max(3, steps // 2) if m >= 2048 else steps
                    us = _time_rotating(weights, m, k, n, qa.MODE_MFMA, reps, max(2, warmup))
                    flops = 2.0 * m * n * k
                    tflops = flops / (us * 1e-6) / 1e12
                    intensity = flops / abytes
                    attainable = min(MFMA_F16_PEAK_TFLOPS, intensity * HBM_PEAK_GBPS / 1e3)
                    # the same point in F32 mode: the split-half GEMM, within the f32 bars
                    us32 = _time_rotating(weights, m, k, n, qa.MODE_F32, reps, max(2, warmup))
                    entry = {"config": cfg_i, "qtype": QNAME[qtype], "m": m, "k": k, "n": n,
                             "us": round(us, 2), "tflops": round(tflops, 1),
                             "roofline": {"bound": "mfma" if intensity >= RIDGE_FLOP_PER_BYTE else "hbm",
                                          "achieved": round(tflops, 1), "peak": round(attainable, 1),
                                          "unit": "TFLOP/s", "frac": round(tflops / attainable, 4),
                                          "frac_of_f16_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                                          "intensity_flop_per_byte": round(intensity, 1)},
                             "f32_mode": {"us": round(us32, 2), "tflops": round(flops / (us32 * 1e-6) / 1e12, 1),
                                          "kernel": "split-half GEMM (token-identical prompts)"}}
                    if with_cpu:
                        entry["cpu_baseline"] = _cpu_point(qtype, k, n, m, blocks, "TFLOP/s", flops)
                out[kind].append(entry)
                print(f"bench configs: {kind} {QNAME[qtype]} M={m} K={k} N={n}: "
                      f"{entry['us']} us, frac {entry['roofline']['frac']}", file=sys.stderr, flush=True)
            for w in weights:
                w.free()
    out["device"] = ctx.device_name()
    ctx.close()
    out["note"] = ("GEMV: F32 mode, us per call over resident weight copies (>= 512 MB); gemv_row_major: "
                   "the same on row-major (blocks along N) weights, the tiled row-major image; GEMM: MFMA mode, "
                   "f16 activation conversion + GEMM per call (f32_mode: the same point in F32 mode, "
                   "the split-half GEMM); roofline.frac of the GEMM is against "
                   "min(f16 peak, intensity x HBM peak); cpu_baseline: scalar CpuScalar port and, for "
                   "Q8_0/Q4_0, the cpu-simd block dot, one pinned core, in the unit of the point")
    return out


# --------------------------------------------------------------- e2e decode

E2E_PROMPT, E2E_NEW = 512, 128
E2E_GOLDEN = os.path.join(ROOT, "tests", "golden", "qwen3_8b_greedy.json")


def e2e_shapes(cfg):
    """(name, K, N) of the seven projections of one layer."""
    H, I = cfg["hidden_size"], cfg["intermediate_size"]
    QS = cfg["num_attention_heads"] * cfg["head_dim"]
    KS = cfg["num_key_value_heads"] * cfg["head_dim"]
    return [("q_proj", H, QS), ("k_proj", H, KS), ("v_proj", H, KS), ("o_proj", QS, H),
            ("gate_proj", H, I), ("up_proj", H, I), ("down_proj", I, H)]


def e2e_step_bytes(cfg, position: int) -> int:
    """HBM bytes one decode step at `position` must move: every layer's Q4_K
    weights and the Q6_K head (wire bytes), the keys and values of positions
    0..position read and one position written (f32), the embedding row and the
    f32 activation rows of each GEMV."""
    H, V = cfg["hidden_size"], cfg["vocab_size"]
    L, hd, kvh = cfg["num_hidden_layers"], cfg["head_dim"], cfg["num_key_value_heads"]
    weights = sum(n * (k // 256) * 144 + (k + n) * 4 for _, k, n in e2e_shapes(cfg))
    kv = (position + 2) * kvh * hd * 4 * 2
    head = V * (H // 256) * 210 + (H + V) * 4
    return L * (weights + kv) + head + H * 4


def e2e_bench(repeats: int = 3, with_cpu: bool = True) -> dict:
    """Qwen3-8B-shape decode tokens/s: build the random-init model of
    quantinfer_amd.synth on the device, then `repeats` x (reset cache,
    512-token prompt, 128 greedy decode steps) in F32 mode (the decoder's
    default), whose ids equal the CPU run's; the decode time is the HIP-event
    time of the decode steps.
    One more run in AUTO mode (f16 GEMM prompt) is reported beside it. Both
    runs' ids are compared with the CPU run's."""
    import numpy as np
    import quantinfer_amd as qa
    from quantinfer_amd import synth

    cfg = dict(synth.QWEN3_8B)
    t0 = time.perf_counter()
    w = synth.qwen3_weights(cfg, synth.DEFAULT_SEED, 3, 5)
    cpu_layer = {name: w["layers"][0][name][2] for name, _, _ in e2e_shapes(cfg)}
    cpu_head = w["head"][2]
    ctx = qa.Context(0)
    model = synth.device_model(ctx, cfg, w)
    del w
    build_s = time.perf_counter() - t0
    cache = model.kv_cache(E2E_PROMPT + E2E_NEW)
    prompt = synth.prompt(cfg, E2E_PROMPT)
    # F32 mode: the configuration whose greedy ids equal the CPU run's (the
    # split-half GEMM for the prompt's Q4_K linears; the decode steps run the
    # f32 GEMV in every mode)
    model.set_mode(qa.MODE_F32)
    model.generate(cache, prompt, E2E_NEW)  # warm-up: workspaces and the decode graph
    runs, tokens = [], None
    for _ in range(repeats):
        cache.reset()
        out = model.generate(cache, prompt, E2E_NEW)
        t = model.last_timing()
        if tokens is not None and out != tokens:
            raise RuntimeError("decode is not deterministic across runs")
        tokens = out
        runs.append((t.decode_ms, t.prefill_ms, t.decode_steps))
    # AUTO mode: the f16-operand GEMM for the prompt (faster prefill, not
    # token-identical at this config's near-ties)
    model.set_mode(qa.MODE_AUTO)
    cache.reset()
    model.generate(cache, prompt, E2E_NEW)
    cache.reset()
    tokens_auto = model.generate(cache, prompt, E2E_NEW)
    auto_timing = model.last_timing()
    device = ctx.device_name()
    cache.free()
    model.free()
    ctx.close()
    golden = None
    if os.path.exists(E2E_GOLDEN):
        with open(E2E_GOLDEN) as f:
            g = json.load(f)
        if g["prompt"] == [int(v) for v in prompt] and g["seed"] == synth.DEFAULT_SEED:
            golden = g["tokens"]

    def match(ids):
        if golden is None:
            return None
        first = next((i for i, (a, b) in enumerate(zip(ids, golden)) if a != b), None)
        return {"equal": first is None and len(ids) == len(golden), "first_difference": first,
                "equal_ids": sum(a == b for a, b in zip(ids, golden)), "of": len(golden)}

    decode_ms = statistics.median(r[0] for r in runs)
    prefill_ms = statistics.median(r[1] for r in runs)
    steps = runs[0][2]
    ms_tok = decode_ms / steps
    tok_s = 1e3 / ms_tok
    avg_bytes = sum(e2e_step_bytes(cfg, E2E_PROMPT + i) for i in range(steps)) / steps
    achieved = avg_bytes / (ms_tok * 1e-3) / 1e9
    return {
        "metric": "Qwen3-8B-shape decode tok/s",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps,
        "warmup": 1, "ms_per_step": round(ms_tok, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 activations, Q4_K linears (Q6_K head), f32 KV cache",
        "data": "synthetic random-init model (quantinfer_amd.synth): N(0,0.02^2) weights quantized to "
                "Q4_K (head Q6_K) by qi_hip_quantize, N(0,0.02^2) f32 embedding, N(1,0.05^2) norms; "
                "uniform random prompt ids",
        "config": {"workload": "qwen3_8b_shape_decode_prompt512_new128", "layers": 36,
                   "hidden": 4096, "heads": 32, "kv_heads": 8, "head_dim": 128,
                   "intermediate": 12288, "vocab": 151936, "prompt_tokens": E2E_PROMPT,
                   "decode_steps": steps, "mode": "f32, the default (split-half matrix-core GEMM for the prompt, f32 GEMV for the decode steps)",
                   "repeats": repeats, "device": device},
        "prefill_tok_s": round(E2E_PROMPT / (prefill_ms * 1e-3), 1),
        "prefill_ms": round(prefill_ms, 3),
        "model_build_s": round(build_s, 1),
        "tokens_vs_cpu_run": {"f32": match(tokens), "auto": match(tokens_auto),
                              "reference": "tests/golden/qwen3_8b_greedy.json (oracle CpuScalar run)"},
        "auto_mode": {"note": "f16-operand MFMA GEMM for the prompt; decode steps unchanged",
                      "prefill_ms": round(auto_timing.prefill_ms, 3),
                      "prefill_tok_s": round(E2E_PROMPT / (auto_timing.prefill_ms * 1e-3), 1),
                      "decode_tok_s": round(1e3 * auto_timing.decode_steps / auto_timing.decode_ms, 2)},
        "roofline": {"bound": "hbm", "scope": "one whole decode step (all kernels of a token)",
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "bytes_per_step": int(avg_bytes), "traffic": None},
        "cpu_baseline": e2e_cpu_baseline(cfg, cpu_layer, cpu_head) if with_cpu else None,
    }


def e2e_cpu_baseline(cfg, layer: dict, head_blocks) -> dict:
    """The oracle's CpuScalar port on one pinned core, on a bounded sample:
    the seven Q4_K output-row matmuls of one layer at M=1 and the f32 LM head
    (the reference dequantizes a Q6_K head to f32 at load,
    runtime/src/qwen3/loader.rs:47-61), scaled to 36 layers per token.
    Attention and the norms (under 1% of the work) are left out."""
    from oracle import pyoracle as po

    H, V = cfg["hidden_size"], cfg["vocab_size"]
    head = po.dequantize(5, head_blocks).reshape(V, H)
    try:
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {min(old)})
    except (AttributeError, OSError):
        old = None
    try:
        t_layer = 0.0
        for name, k, n in e2e_shapes(cfg):
            x = normal(0x5EED8000, k).reshape(1, k)
            t = time.perf_counter()
            po.matmul_output_rows(3, x, layer[name], n)
            t_layer += time.perf_counter() - t
        x = normal(0x5EED8001, H).reshape(1, H)
        t = time.perf_counter()
        po.linear_rows(x, head, 1)
        t_head = time.perf_counter() - t
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    sec = cfg["num_hidden_layers"] * t_layer + t_head
    del head
    return {"value": round(1.0 / sec, 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"one layer's 7 Q4_K projections ({t_layer:.2f} s) x36 + f32 LM head "
                      f"({t_head:.2f} s) at M=1: {sec:.1f} s per decode token; oracle C port of "
                      f"CpuScalar (matmul.rs:282-332, :92-117), 1 pinned core of {host_cpu()}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20,
                    help="timed steps (a step is one GEMV over each resident weight copy)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="time device-to-device copies of 256 MiB instead (counter calibration)")
    ap.add_argument("--workload", choices=["gemv", "gemm", "e2e", "f32head", "configs", "calib", "timeline",
                                           "libgemm"],
                    default="gemv",
                    help="gemv: the headline decode GEMV with the Q8_0 GEMV, the GEMMs and the e2e "
                         "decode line embedded (default); gemm: one MFMA prefill GEMM; e2e: "
                         "Qwen3-8B-shape decode only; calib: streaming-read ceilings (measurement "
                         "aid); timeline: the M=1 GEMV's workgroup timeline (profiling build); "
                         "libgemm: the GEMM shape as a plain f16 library GEMM, for scale")
    ap.add_argument("--no-e2e", action="store_true", help="gemv: leave out the e2e decode run")
    ap.add_argument("--no-gemm", action="store_true", help="gemv: leave out the GEMM objects")
    ap.add_argument("--no-abi", action="store_true",
                    help="gemv: leave out the through-ABI calls (host buffers), so a kernel trace holds "
                         "only the timed device launches")
    ap.add_argument("--no-f32head", action="store_true", help="gemv: leave out the F32 LM-head object")
    ap.add_argument("--no-configs", action="store_true",
                    help="gemv: leave out the table of every BASELINE config point")
    ap.add_argument("--cpu-simd", action="store_true",
                    help="only the CPU table: scalar and cpu-simd Q8_0/Q4_0 kernels, one core")
    ap.add_argument("--qtype", default="q4_k", help="gemv/gemm: q8_0, q4_0, q4_k, q5_k or q6_k")
    ap.add_argument("--layout", choices=["output_rows", "row_major"], default="output_rows",
                    help="gemv: the weight layout (row_major: QuantInfer blocks along N, the GEMV alone)")
    ap.add_argument("--mode", choices=["mfma", "f32"], default="mfma",
                    help="gemm: the f16-operand GEMM (mfma) or F32 mode's split-half GEMM (f32; Q4_K/Q5_K)")
    ap.add_argument("--mkn", default=None,
                    help="M,K,N (gemm default 2048,4096,12288; gemv default 1,4096,14336)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); "
              "the multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration(args.steps)
        return
    if args.cpu_simd:
        print(json.dumps(cpu_simd_table()))
        return
    qt = {"q8_0": 1, "q4_0": 2, "q4_k": 3, "q5_k": 4, "q6_k": 5}[args.qtype]
    if args.workload == "gemm":
        m, k, n = (int(v) for v in (args.mkn or "2048,4096,12288").split(","))
        print(json.dumps(gemm_bench(qt, m, k, n, max(args.steps, 20), args.warmup, args.mode)))
        return
    if args.workload == "e2e":
        print(json.dumps(e2e_bench(with_cpu=not args.no_cpu)))
        return
    if args.workload == "configs":
        print(json.dumps(configs_table(args.steps, args.warmup, not args.no_cpu)))
        return
    if args.workload == "f32head":
        print(json.dumps(f32_head_bench(args.steps, args.warmup)))
        return
    if args.workload == "libgemm":
        m, k, n = (int(v) for v in (args.mkn or "2048,4096,12288").split(","))
        out = library_f16_gemm(m, k, n, max(args.steps, 20))
        out.update({"m": m, "k": k, "n": n})
        print(json.dumps(out))
        return
    if args.workload == "calib":
        print(json.dumps(calib_bench(args.steps)))
        return
    if args.workload == "timeline":
        m, k, n = (int(v) for v in (args.mkn or f"{M},{K},{N}").split(","))
        if not 1 <= m <= 16:
            sys.exit("bench.py --workload timeline: the stamps cover the decode GEMV (M <= 16)")
        print(json.dumps(timeline_bench(qtype=qt, k=k, n=n, m=m)))
        return

    m, k, n = (int(v) for v in (args.mkn or f"{M},{K},{N}").split(","))
    rm = args.layout == "row_major"
    g = gemv_bench(qt, k, n, m, args.steps, args.warmup, with_abi=not args.no_abi, row_major=rm)
    line = gemv_line(qt, k, n, m, g, args.steps, args.warmup, row_major=rm)
    if not rm:
        line["metric"] = "quant GEMV GB/s (% of HBM peak) at 4096x14336; Qwen3-8B-shape decode tok/s"
    line["cpu_baseline"] = None if args.no_cpu or (m, k, n) != (M, K, N) or rm else cpu_baseline(qt)
    abytes = algorithmic_bytes(qt, k, n, m)
    line["through_abi"] = None if args.no_abi else {
        "value": round(abytes / (g["abi_ms"] * 1e-3) / 1e9, 2), "unit": "GB/s",
        "ms_per_call": round(g["abi_ms"], 5), "calls": g["abi_calls"],
        "note": "qi_hip_linear with host x and y (H2D, GEMV, D2H, synchronous): the "
                "PCIe-inclusive KernelBackend call, median over calls; not `value`",
    }
    if (qt, m, k, n) == (3, M, K, N) and not rm:
        g8 = gemv_bench(1, K, N, M, args.steps, args.warmup)
        line["gemv_q8_0"] = gemv_line(1, K, N, M, g8, args.steps, args.warmup)
        if not args.no_cpu:
            line["gemv_q8_0"]["cpu_baseline"] = _cpu_point(1, K, N, M, weight_blocks(1, K, N, seed=0x5EED0001),
                                                           "GB/s", algorithmic_bytes(1, K, N, M))
        if not args.no_f32head:
            line["f32_matmul_head"] = f32_head_bench(args.steps, args.warmup)
        if not args.no_gemm:
            # the GEMM objects take their own counts: 20 warm-up calls (about
            # 6 ms, so that the clocks settle) and 50 timed ones
            line["gemm"] = {QNAME[q]: gemm_bench(q, 2048, 4096, 12288, 50, 20) for q in (3, 1)}
            # F32 mode at the same shape: the split-half GEMM (token-identical prompts)
            line["gemm_f32"] = {"q4_k": gemm_bench(3, 2048, 4096, 12288, 20, 5, "f32")}
        if not args.no_configs:
            line["configs"] = configs_table(min(args.steps, 10), min(args.warmup, 3), not args.no_cpu)
        if not args.no_e2e:
            line["e2e"] = e2e_bench(with_cpu=not args.no_cpu)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
