"""Benchmark of the quantized GEMM path on one MI355X.

Headline metric: INT8 TOPS at M=N=K=8192 + HBM GB/s of the M=1 decode
GEMV (N=14336, K=4096).  One "step" is one W8A8 INT8 GEMM at 8192^3 (per-token x
per-channel fp32 scales, fp32 out) with inputs resident in HBM; `value` is its
throughput in TOPS.  The decode GEMV (bf16 out + fused bias, weights rotated
over 8 distinct 56 MiB buffers so the 256 MiB MALL cannot hold them) is timed in
the same run and reported under "decode_gemv", and the M=16 decode (the other
end of the decode configs) under "decode_gemv_m16", and a 64-row batch on the
same weights (the batched decode kernel) under "decode_batch_m64".  Beside
them, "hbm_read_floor" is the fastest plain read of the same 56 MiB on the same
box (a kernel that only loads, several grid shapes), and each decode line's
"of_read_floor" is that time over its own.  The other
two GEMM configurations of the benchmark set sit in the same line with their
own rooflines: "c3" (prefill 4096x11008x4096, bf16 out) and "c5" (FP8 e4m3
8192^3, B [K,N] as the reference's launcher reads it, operands drawn as fp32
N(0,1) and quantised at per-tensor amax/448).  Inputs are random (torch RNG
on the device), never zero-filled.

Each GEMM configuration first runs back to back for a fixed wall time
(--preheat-ms): the shader clock settles over the first ~50 ms of sustained
MFMA load (measured: 481 us per launch over the first 100 launches of the
headline GEMM, 430 us after), and the counted warm-up steps alone are too few
to cover that.  The shader clock under the headline load is read through
amdsmi and reported as "sclk_mhz" (with the socket power: this GEMM runs at
the board's power limit, so the clock is the box-to-box variable).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--extra | --fp8 --swiglu --half --batch --shards
       --decode-families] [--vendor] [--data-sweep] [--no-cpu] [--preheat-ms MS] [--clock-ms MS]
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "flash-kernel-engine_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_INT8_TOPS = 5000.0   # MI355X dense INT8 MFMA, published (5.0 POP/s)
PEAK_FP8_TFLOPS = 5000.0  # MI355X dense FP8 MFMA, published
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 MFMA, published
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, published (8 TB/s)
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic.json")


# FKE_PATH_MFMA_* (include/fke_qgemm.h) -> tile name
TILE_LABELS = {5: "256x256", 6: "128x128", 7: "128x128_ring4", 8: "128x64_ring4", 9: "64x64_ring4"}


def gemv_kernel(L, _lib, M, N=14336, K=4096, layout="nk"):
    """Kernel the dispatcher picks for an M-row INT8 batch (K % 4096 == 0, B [N,K] or [K,N]): the
    decode family's, or the MFMA GEMM's with its tile."""
    code = _lib.B_NK if layout == "nk" else _lib.B_KN
    path = L.fke_select_path_i8(4096, 4096, 4096, M, N, K, _lib.OUT_BF16, code)
    if path == _lib.PATH_MFMA:
        tile = TILE_LABELS[L.fke_select_mfma_tile(M, N, K, code, 0, 0)]
        return f"gemm_mfma_kernel<i8,{layout.upper()},bf16,{tile}>"
    if layout == "kn":
        first = "gemv_kn_row_kernel<i8>" if M == 1 else "gemv_kn_split_kernel<i8>"
        return first + "+kn_reduce_kernel<i8,bf16>"
    return "gemv_rows_kernel" if M <= 2 else "gemv_lds_kernel"


def traffic(key):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE + WRITE_SIZE (calibrated
    against a copy kernel), as recorded in profiles/traffic.json; None if absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f).get(key)
    except (OSError, ValueError):
        return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # ~50 ms of warm-up: the first ~50-100 ms of sustained MFMA load run at a
    # lower, still-settling clock (measured 558 us/step there vs 505 after).
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--preheat-ms", type=float, default=250.0,
                    help="wall time each GEMM configuration runs back to back before its counted warm-up")
    ap.add_argument("--clock-ms", type=float, default=1100.0,
                    help="wall time the headline GEMM keeps running after its timed steps for the clock readings "
                         "(the metrics refresh once a second; 0 skips them)")
    ap.add_argument("--gemv-buffers", type=int, default=8)
    ap.add_argument("--gemv-launches", type=int, default=400)
    ap.add_argument("--extra", action="store_true", help="also time configs 2 and 4, decode M=4 and batched decode M=32,64,128")
    ap.add_argument("--swiglu", action="store_true", help="also time the SwiGLU configs (part of --extra)")
    ap.add_argument("--half", action="store_true", help="also time the fp16/bf16 GEMM (part of --extra)")
    ap.add_argument("--fp8", action="store_true", help="also time the FP8 e4m3 GEMM 8192^3 (part of --extra)")
    ap.add_argument("--batch", action="store_true",
                    help="also time batched decode M=32,64,128 on the decode weights (part of --extra)")
    ap.add_argument("--decode-families", action="store_true",
                    help="also time decode M=1,2,4,8,16 on the MFMA kernels the dispatcher picks and on the "
                         "VALU dot-product kernels (FKE_PATH_GEMV_DOT), for the choice between them")
    ap.add_argument("--ksplit", action="store_true",
                    help="also time the MFMA GEMM's K split on few-tile shapes with a long K beside the unsplit tile "
                         "(part of --extra)")
    ap.add_argument("--shards", action="store_true",
                    help="also time the per-GPU shards of 8-way tensor parallelism (part of --extra)")
    ap.add_argument("--tile-sweep", action="store_true",
                    help="also time every MFMA GEMM tile (256x256, 128x128, and the 4-stage rings) on shapes around the dispatcher's "
                         "tile rule, INT8, FP8 and bf16 (B [N,K]), beside the tile it picks")
    ap.add_argument("--data-sweep", action="store_true",
                    help="also time the headline GEMM on zero, constant and narrow-range operands (clock vs data)")
    ap.add_argument("--odd-k", action="store_true",
                    help="prefill shapes with K %% 128 != 0 (4096x11008x4160, 4096x4096x2880) on the MFMA GEMM "
                         "(partial last stage), 4096x11008x4100 on the INT8 word kernel, each also on the "
                         "any-shape generic kernel (part of --extra)")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="the INT8 matrix-core ceiling: a register-only v_mfma_i32_32x32x32_i8 stream "
                         "(libfke_probe.so) on the headline's operand distribution and on constant operands, "
                         "with the shader clock and socket power while it runs")
    ap.add_argument("--vendor", action="store_true",
                    help="also time the vendor library (hipBLASLt through torch) on the 8192^3 GEMMs, for context")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 512 MiB device copy (reference kernel for FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus above 1 is not supported "
                                   "(the quantized GEMM path has no multi-GPU component here)"}))
        sys.exit(2)

    import torch

    from flash_engine import _lib

    L = _lib.lib()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)

    def rand_i8(*shape):
        return torch.randint(-127, 128, shape, dtype=torch.int8, device=dev, generator=gen)

    def rand_u(n, lo=0.001, hi=0.02):
        return torch.rand(n, device=dev, generator=gen) * (hi - lo) + lo

    def timed(fn, n, warm, preheat_ms=0.0):
        if preheat_ms > 0:
            preheat(torch, fn, preheat_ms)
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n  # ms per call

    # ---- headline: INT8 GEMM 8192^3, fp32 out --------------------------------
    M = N = K = 8192
    A, B = rand_i8(M, K), rand_i8(N, K)
    sa, sb = rand_u(M), rand_u(N)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)

    def gemm():
        st = L.fke_qgemm_i8(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, sa.data_ptr(),
                            sb.data_ptr(), 1.0, 1.0, None, _lib.OUT_F32, _lib.B_NK, sh)
        if st:
            raise RuntimeError(f"fke_qgemm_i8 failed: {_lib.status_string(st)}")

    torch.cuda.synchronize()
    clock = ClockSampler() if args.clock_ms > 0 else None
    if clock:
        clock.start()
    pre_n, pre_ms = preheat(torch, gemm, args.preheat_ms) if args.preheat_ms > 0 else (0, 0.0)
    t0 = time.perf_counter()
    ms = timed(gemm, args.steps, args.warmup)
    wall = time.perf_counter() - t0
    if clock:
        preheat(torch, gemm, args.clock_ms)  # the same load a while longer: the metrics refresh once a second
    sclk = clock.stop() if clock else {"value": None, "error": "not sampled (--clock-ms 0)"}
    ops_per = 2.0 * M * N * K
    tops = ops_per / (ms * 1e-3) / 1e12
    del C

    # ---- C3 prefill and C5 FP8 square, each with its own roofline -------------
    c3 = c3_line(torch, L, _lib, dev, rand_i8, rand_u, timed, args)
    c5 = c5_line(torch, L, _lib, dev, gen, timed, args)

    # ---- decode GEMV M=1 and M=16, N=14336, K=4096, bf16 out + bias -------------
    gemv = gemv_bench(torch, L, _lib, dev, gen, 1, args.gemv_buffers, args.gemv_launches)
    gemv16 = gemv_bench(torch, L, _lib, dev, gen, 16, args.gemv_buffers, args.gemv_launches)
    batch64 = gemv_bench(torch, L, _lib, dev, gen, 64, args.gemv_buffers, args.gemv_launches)
    # the same decode with B stored [K,N], the layout of the reference's Python op
    gemv_kn1 = gemv_bench(torch, L, _lib, dev, gen, 1, args.gemv_buffers, args.gemv_launches, layout="kn")
    gemv_kn16 = gemv_bench(torch, L, _lib, dev, gen, 16, args.gemv_buffers, args.gemv_launches, layout="kn")
    # the fastest plain read of the same weight bytes on this box, and each decode line against it
    floor = read_floor(torch, dev, gen, 14336 * 4096, args.gemv_buffers, args.gemv_launches)
    for d in (gemv, gemv16, gemv_kn1, gemv_kn16):
        d["read_floor_us"] = floor["us"]
        d["of_read_floor"] = round(floor["us"] / d["us_per_launch"], 4)

    line = {
        "metric": "INT8 TOPS at 8192^3 + HBM GB/s at M=1 decode GEMV (N=14336,K=4096)",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (uniform int8 [-127,127], fp32 scales U[0.001,0.02], device RNG)",
        "config": {"workload": "W8A8 INT8 GEMM M=N=K=8192, B [N,K], per-token x per-channel "
                               "fp32 scales, fp32 out (the square headline workload)",
                   "M": M, "N": N, "K": K, "out": "fp32", "kernel": "gemm_mfma_kernel<i8,NK,f32>"},
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TOP/s", "frac": round(tops / PEAK_INT8_TOPS, 4),
                     "traffic": traffic("gemm_mfma_kernel<i8,NK,f32> M=N=K=8192"),
                     "algorithmic_ops_per_launch": ops_per},
        "preheat_ms": round(pre_ms, 1),
        "preheat_launches": pre_n,
        "sclk_mhz": sclk,
        "c3": c3,
        "c5": c5,
        "decode_gemv": gemv,
        "decode_gemv_m16": gemv16,
        "decode_batch_m64": batch64,
        "decode_gemv_b_kn": gemv_kn1,
        "decode_gemv_m16_b_kn": gemv_kn16,
        "hbm_read_floor": floor,
        "timed_wall_s": round(wall, 3),
    }
    line["hbm_copy_GBps"] = copy_bandwidth(torch, dev, gen)
    if args.calibrate_copy:
        src = torch.randint(0, 255, (512 << 20,), dtype=torch.uint8, device=dev, generator=gen)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.extra:
        line["extra"] = extra_configs(torch, L, _lib, dev, gen, timed, rand_i8, rand_u, args)
    elif (args.swiglu or args.half or args.fp8 or args.shards or args.batch or args.decode_families or args.ksplit
          or args.odd_k):
        line["extra"] = {}
        if args.odd_k:
            line["extra"].update(odd_k_configs(torch, L, _lib, dev, timed, rand_i8, rand_u, args))
        if args.ksplit:
            line["extra"].update(ksplit_configs(torch, L, _lib, dev, gen, args))
        if args.decode_families:
            line["extra"].update(decode_family_configs(torch, L, _lib, dev, gen, args))
        if args.batch:
            line["extra"].update(batch_configs(torch, L, _lib, dev, gen, args))
        if args.shards:
            line["extra"].update(shard_configs(torch, L, _lib, dev, gen, timed, rand_i8, rand_u, args))
        if args.fp8:
            line["extra"].update(fp8_configs(torch, L, _lib, dev, gen, timed, args))
        if args.swiglu:
            line["extra"].update(swiglu_configs(torch, L, _lib, dev, gen, timed, rand_i8, rand_u, args))
        if args.half:
            line["extra"].update(half_configs(torch, L, _lib, dev, gen, timed, args))
    if args.vendor:
        line["vendor_context"] = vendor_configs(torch, dev, gen, timed, args)
    if args.data_sweep:
        line["data_sweep"] = data_sweep(torch, L, _lib, dev, gen, timed, args)
    if args.mfma_ceiling:
        line["mfma_ceiling"] = mfma_ceiling(torch, dev, gen, timed, args)
    if args.tile_sweep:
        line["tile_sweep"] = tile_sweep(torch, L, _lib, dev, gen, timed, args)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


def preheat(torch, fn, ms, chunk=16):
    """Run fn back to back until `ms` milliseconds of wall time have passed
    (synchronising every `chunk` launches); returns (launches, wall ms)."""
    t0 = time.perf_counter()
    n = 0
    while True:
        for _ in range(chunk):
            fn()
        torch.cuda.synchronize()
        n += chunk
        el = (time.perf_counter() - t0) * 1e3
        if el >= ms:
            return n, el


class ClockSampler:
    """Reads the GPU's shader clock and socket power through amdsmi on a
    background thread (every 5 ms) while the headline GEMM runs.  The
    firmware refreshes its metrics table about once a second (measured: the
    table's system_clock_counter steps by 1e9 ns), so only readings whose
    counter advanced while the load ran - at least 100 ms after it started -
    count; the clock is the mean over the XCDs of current_gfxclks."""

    def __init__(self, period=0.005):
        self.period = period
        self.fresh = []
        self.t_load = None
        self.err = None
        self._stop = False
        self._th = None
        self._last = None
        try:
            import amdsmi
            amdsmi.amdsmi_init()
            self.smi = amdsmi
            self.h = amdsmi.amdsmi_get_processor_handles()[0]
            self._last = self._read()[0]
        except Exception as e:  # no amdsmi or no permission: report why
            self.smi = None
            self.err = repr(e)[:160]

    def _read(self):
        m = self.smi.amdsmi_get_gpu_metrics_info(self.h)
        xs = [v for v in m.get("current_gfxclks", []) if isinstance(v, (int, float))]
        power = m.get("current_socket_power")
        return (m.get("system_clock_counter"), sum(xs) / len(xs) if xs else None, min(xs) if xs else None,
                max(xs) if xs else None, power if isinstance(power, (int, float)) else None)

    def _run(self):
        while not self._stop:
            try:
                r = self._read()
                if r[0] != self._last:
                    self._last = r[0]
                    if r[1] is not None and time.perf_counter() - self.t_load >= 0.1:
                        self.fresh.append(r)
            except Exception as e:
                self.err = repr(e)[:160]
            time.sleep(self.period)

    def start(self):
        self.t_load = time.perf_counter()
        if self.smi is not None:
            import threading
            self._th = threading.Thread(target=self._run, daemon=True)
            self._th.start()

    def stop(self):
        self._stop = True
        if self._th is not None:
            self._th.join()
        if self.smi is None or not self.fresh:
            return {"value": None, "error": self.err or "no metrics refresh during the load"}
        clk = [r[1] for r in self.fresh]
        pw = [r[4] for r in self.fresh if r[4] is not None]
        return {"value": round(sum(clk) / len(clk), 1),
                "xcd_min": min(r[2] for r in self.fresh), "xcd_max": max(r[3] for r in self.fresh),
                "socket_power_w": round(sum(pw) / len(pw), 1) if pw else None, "readings": len(clk),
                "source": "amdsmi gpu_metrics current_gfxclks (mean over XCDs), readings refreshed while the "
                          "headline GEMM ran back to back (pre-heat, timed steps, then 1.1 s more)"}


def c3_line(torch, L, _lib, dev, rand_i8, rand_u, timed, args):
    """W8A8 prefill M=4096 N=11008 K=4096 (MLP up), int8
    uniform, per-token x per-channel scales U[0.001,0.02], bf16 out."""
    M, N, K = 4096, 11008, 4096
    sh = torch.cuda.current_stream(dev).cuda_stream
    A, B, sa, sb = rand_i8(M, K), rand_i8(N, K), rand_u(M), rand_u(N)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def run():
        st = L.fke_qgemm_i8(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, sa.data_ptr(), sb.data_ptr(), 1.0,
                            1.0, None, _lib.OUT_BF16, _lib.B_NK, sh)
        if st:
            raise RuntimeError(f"fke_qgemm_i8 failed: {_lib.status_string(st)}")

    ms = timed(run, args.steps, args.warmup, args.preheat_ms)
    ops = 2.0 * M * N * K
    t = ops / (ms * 1e-3) / 1e12
    del A, B, C
    return {"metric": "INT8 TOPS, prefill W8A8 GEMM M=4096 N=11008 K=4096 (bf16 out)", "value": round(t, 1),
            "unit": "TOPS", "ms_per_launch": round(ms, 4), "steps": args.steps,
            "roofline": {"bound": "mfma", "achieved": round(t, 1), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                         "frac": round(t / PEAK_INT8_TOPS, 4),
                         "traffic": traffic("gemm_mfma_kernel<i8,NK,bf16> M=4096 N=11008 K=4096"),
                         "algorithmic_ops_per_launch": ops},
            "kernel": "gemm_mfma_kernel<i8,NK,bf16>"}


def c5_line(torch, L, _lib, dev, gen, timed, args):
    """FP8 e4m3 8192^3.  A and B are drawn as fp32 N(0,1) and
    quantised to e4m3 with per-tensor scales amax/448 (saturating; the largest
    element maps to 448), B stored [K,N] as the reference's launcher reads it
    (src/quantized_gemm.cu:113), fp32 accumulation, bf16 out."""
    M = N = K = 8192
    sh = torch.cuda.current_stream(dev).cuda_stream

    def quant(shape):
        x = torch.randn(shape, device=dev, generator=gen)
        s = float(x.abs().max()) / 448.0
        q = torch.clamp(x / s, -448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
        del x
        return q.contiguous(), s

    A8, s_a = quant((M, K))
    B8, s_b = quant((K, N))
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def run():
        st = L.fke_qgemm_f8(A8.data_ptr(), B8.data_ptr(), C.data_ptr(), M, N, K, s_a, s_b, None, _lib.OUT_BF16,
                            _lib.B_KN, sh)
        if st:
            raise RuntimeError(f"fke_qgemm_f8 failed: {_lib.status_string(st)}")

    ms = timed(run, args.steps, args.warmup, args.preheat_ms)
    flops = 2.0 * M * N * K
    t = flops / (ms * 1e-3) / 1e12
    del A8, B8, C
    return {"metric": "FP8 TFLOPS, scaled e4m3 GEMM M=N=K=8192, B [K,N] (bf16 out)", "value": round(t, 1),
            "unit": "TFLOPS", "ms_per_launch": round(ms, 4), "steps": args.steps,
            "data": "fp32 N(0,1) quantised to e4m3 at per-tensor amax/448 on the device",
            "roofline": {"bound": "mfma", "achieved": round(t, 1), "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(t / PEAK_FP8_TFLOPS, 4),
                         "traffic": traffic("gemm_mfma_kernel<f8,KN,bf16> M=N=K=8192"),
                         "algorithmic_flops_per_launch": flops},
            "kernel": "gemm_mfma_kernel<f8,KN,bf16>"}


def copy_bandwidth(torch, dev, gen):
    """Device-to-device copy of 1 GiB (read + write counted), the achievable
    streaming rate beside the 8.0 TB/s specification."""
    src = torch.randint(0, 255, (1 << 30,), dtype=torch.uint8, device=dev, generator=gen)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    gbs = 2.0 * (1 << 30) * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    return round(gbs, 1)


def read_floor(torch, dev, gen, nbytes, nbuf, launches):
    """The fastest plain read of `nbytes` this box sustains: a kernel that only
    loads (csrc/probe_read.hip: 1 KiB per load instruction, non-temporal, one
    folded value per lane kept live, nothing stored), on `nbuf` rotating random
    buffers from a HIP graph of `launches` launches like the decode lines, over a
    few grid shapes - the decode row kernel's (one 4 KiB block per wave, two
    waves per workgroup), one 8 KiB block per wave, and persistent grids of one
    or two workgroups per CU.  The decode GEMV reads its weights once, so this
    is the attainable floor beside the 8.0 TB/s specification."""
    import ctypes as ct
    P = ct.CDLL(os.path.join(PKG, "lib", "libfke_probe.so"))
    P.fke_probe_read_out_elems.argtypes = [ct.c_int, ct.c_int]
    P.fke_probe_read_out_elems.restype = ct.c_size_t
    P.fke_probe_read.argtypes = [ct.c_void_p, ct.c_int64, ct.c_void_p, ct.c_int, ct.c_int, ct.c_int, ct.c_int32,
                                 ct.c_void_p]
    P.fke_probe_read.restype = ct.c_int
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    bufs = [torch.randint(-127, 128, (nbytes,), dtype=torch.int8, device=dev, generator=gen) for _ in range(nbuf)]
    kib = nbytes // 1024
    shapes = {"4KiB_per_wave_2_waves": (4, 2, kib // 8), "8KiB_per_wave_4_waves": (8, 4, kib // 32),
              "persistent_2_per_cu_4_waves": (8, 4, 2 * cus), "persistent_1_per_cu_8_waves": (8, 8, cus)}
    res = {"bytes": nbytes, "buffers": nbuf}
    best = None
    for name, (unit, waves, grid) in shapes.items():
        out = torch.empty(P.fke_probe_read_out_elems(grid, waves), dtype=torch.int32, device=dev)

        def launch(i, st, unit=unit, waves=waves, grid=grid, out=out):
            r = P.fke_probe_read(bufs[i % nbuf].data_ptr(), nbytes, out.data_ptr(), grid, waves, unit, 0x7F7F7F7F, st)
            if r:
                raise RuntimeError(f"fke_probe_read failed: status {r}")
        us = graph_us(torch, dev, launch, launches, 2 * nbuf)
        res[name] = round(us, 3)
        best = us if best is None else min(best, us)
    res["us"] = round(best, 3)
    res["GB/s"] = round(nbytes / best / 1e3, 1)
    res["frac_of_spec"] = round(nbytes / best / 1e3 / PEAK_HBM_GBS, 4)
    del bufs
    return res


def gemv_bytes(M, N, K, out_bytes=2, bias=True):
    return M * K + N * K + 4 * M + 4 * N + (4 * N if bias else 0) + out_bytes * M * N


def graph_us(torch, dev, launch, launches, warm, reps=3, windows=3, detail=None):
    """Per-launch microseconds of `launch(i, stream)` captured `launches` times in
    one HIP graph: `windows` timed windows of `reps` replays each (events on the
    graph's stream), their median returned and every window's figure appended to
    `detail` when given.  (The boxes now and then run a few milliseconds of HBM
    traffic about 30 % slower, every kernel alike; the median keeps one such
    window from setting the figure.)"""
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):  # warm up outside the graph
        for i in range(warm):
            launch(i, s.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(launches):
            launch(i, s.cuda_stream)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        g.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(windows):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):  # replay on s, where the events are recorded
            e0.record(s)
            for _ in range(reps):
                g.replay()
            e1.record(s)
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1e3 / (reps * launches))
    if detail is not None:
        detail.extend(round(x, 3) for x in per)
    return sorted(per)[len(per) // 2]


def eager_us(torch, dev, launch, launches):
    """Per-call microseconds of `launches` eager calls through the C ABI (ctypes
    call, argument checks, dispatch and launch on the current stream, no graph),
    events around them as in the reference's benchmark idiom
    (benchmarks/bench_decoding.cu:33-58)."""
    sh = torch.cuda.current_stream(dev).cuda_stream
    for i in range(16):
        launch(i, sh)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(launches):
        launch(i, sh)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / launches


def decode_family_configs(torch, L, _lib, dev, gen, args, N=14336, K=4096):
    """Decode on the C2 weights (N = 14336, K = 4096, bf16 out + bias, 8 rotating weights) on the
    family the dispatcher picks (row kernel for M <= 2, LDS-streamed MFMA kernel above) and on the
    VALU dot-product family (row kernel for M <= 4, split-K sdot kernel above), HIP-graph timed."""
    res = {}
    nbuf = args.gemv_buffers
    Bs = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=gen) for _ in range(nbuf)]
    sb = torch.rand(N, device=dev, generator=gen) * 0.019 + 0.001
    bias = torch.randn(N, device=dev, generator=gen) * 0.02
    for M in (1, 2, 4, 8, 16):
        A = torch.clamp(torch.round(torch.randn((M, K), device=dev, generator=gen) * 30), -127, 127).to(torch.int8)
        sa = torch.rand(M, device=dev, generator=gen) * 0.019 + 0.001
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        for name, path in (("auto", _lib.PATH_AUTO), ("dot", _lib.PATH_GEMV_DOT)):
            def launch(i, st, path=path):
                r = L.fke_qgemm_i8_on_path(path, A.data_ptr(), Bs[i % nbuf].data_ptr(), out.data_ptr(), M, N, K,
                                           sa.data_ptr(), sb.data_ptr(), 1.0, 1.0, bias.data_ptr(), _lib.OUT_BF16,
                                           _lib.B_NK, st)
                if r:
                    raise RuntimeError(f"decode failed: {_lib.status_string(r)}")
            us = graph_us(torch, dev, launch, args.gemv_launches, 2 * nbuf)
            nbytes = gemv_bytes(M, N, K)
            res[f"decode_M{M}_{name}"] = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                                          "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4)}
    del Bs
    return res


def gemv_bench(torch, L, _lib, dev, gen, M, nbuf, launches, N=14336, K=4096, layout="nk", path=None):
    """Launch-averaged duration of the decode GEMV from a HIP graph of `launches`
    calls cycling over `nbuf` distinct weight buffers (>= 448 MiB in total);
    B stored [N,K] ("nk") or [K,N] ("kn", the reference's Python-op layout);
    `path` pins a kernel family (FKE_PATH_*) instead of the dispatcher's choice."""
    A = torch.clamp(torch.round(torch.randn((M, K), device=dev, generator=gen) * 30), -127, 127).to(torch.int8)
    shape = (N, K) if layout == "nk" else (K, N)
    code = _lib.B_NK if layout == "nk" else _lib.B_KN
    Bs = [torch.randint(-127, 128, shape, dtype=torch.int8, device=dev, generator=gen) for _ in range(nbuf)]
    sa = torch.rand(M, device=dev, generator=gen) * 0.019 + 0.001
    sb = torch.rand(N, device=dev, generator=gen) * 0.019 + 0.001
    bias = torch.randn(N, device=dev, generator=gen) * 0.02
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def launch(i, sh):
        if path is None:
            st = L.fke_qgemm_i8(A.data_ptr(), Bs[i % nbuf].data_ptr(), out.data_ptr(), M, N, K,
                                sa.data_ptr(), sb.data_ptr(), 1.0, 1.0, bias.data_ptr(), _lib.OUT_BF16,
                                code, sh)
        else:
            st = L.fke_qgemm_i8_on_path(path, A.data_ptr(), Bs[i % nbuf].data_ptr(), out.data_ptr(), M, N, K,
                                        sa.data_ptr(), sb.data_ptr(), 1.0, 1.0, bias.data_ptr(), _lib.OUT_BF16,
                                        code, sh)
        if st:
            raise RuntimeError(f"gemv failed: {_lib.status_string(st)}")

    windows = []
    us = graph_us(torch, dev, launch, launches, 2 * nbuf, detail=windows)
    eager = eager_us(torch, dev, launch, launches)
    nbytes = gemv_bytes(M, N, K)
    gbs = nbytes / (us * 1e-6) / 1e9
    kernel = gemv_kernel(L, _lib, M, N, K, layout)
    if path == _lib.PATH_GEMV and layout == "nk":
        kernel = "gemv_rows_kernel" if M <= 2 else "gemv_lds_kernel"
    return {"metric": f"HBM GB/s, decode GEMV M={M} N={N} K={K}, B {'[N,K]' if layout == 'nk' else '[K,N]'} "
                      f"(bf16 out, fused bias)",
            "value": round(gbs, 1), "unit": "GB/s", "us_per_launch": round(us, 3),
            "us_per_launch_windows": windows, "us_per_call_eager": round(eager, 3),
            "weight_buffers": nbuf, "weight_bytes_cycled": nbuf * N * K,
            "timing": f"HIP graph of {launches} launches, median of 3 windows of 3 replays, events on the "
                      f"graph's stream",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                         "traffic": traffic(f"{kernel} M={M} N={N} K={K} bf16+bias"),
                         "algorithmic_bytes_per_launch": nbytes},
            "kernel": kernel}


def shard_configs(torch, L, _lib, dev, gen, timed, rand_i8, rand_u, args):
    """One GPU's shard of 8-way tensor parallelism, at real size: the decode and prefill
    weights split by output columns (no exchange), and the 8192^3 problem split by columns
    (fp32 out) and by K (int32 partial sums, the exact all-reduce form)."""
    res = {}
    for m in (1, 16):
        r = gemv_bench(torch, L, _lib, dev, gen, m, 48, args.gemv_launches, N=1792, K=4096)
        res[f"tp8_decode_colshard_M{m}_1792x4096_bf16"] = {
            "us": r["us_per_launch"], "GB/s": r["value"], "frac": r["roofline"]["frac"],
            "bytes": r["roofline"]["algorithmic_bytes_per_launch"], "kernel": r["kernel"]}
    sh = torch.cuda.current_stream(dev).cuda_stream
    tiles = TILE_LABELS
    for name, (M, N, K, out, tdt) in {
            "tp8_prefill_colshard_4096x1376x4096_bf16": (4096, 1376, 4096, _lib.OUT_BF16, torch.bfloat16),
            "tp8_int8_colshard_8192x1024x8192_f32": (8192, 1024, 8192, _lib.OUT_F32, torch.float32),
            "tp8_int8_kshard_8192x8192x1024_i32": (8192, 8192, 1024, _lib.OUT_I32, torch.int32),
            "short_prefill_512x14336x4096_bf16": (512, 14336, 4096, _lib.OUT_BF16, torch.bfloat16)}.items():
        A, B, sa, sb = rand_i8(M, K), rand_i8(N, K), rand_u(M), rand_u(N)
        C = torch.empty((M, N), dtype=tdt, device=dev)
        ms = timed(lambda: L.fke_qgemm_i8(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, sa.data_ptr(),
                                          sb.data_ptr(), 1.0, 1.0, None, out, _lib.B_NK, sh),
                   args.steps, args.warmup, args.preheat_ms)
        t = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        tile = L.fke_select_mfma_tile(M, N, K, _lib.B_NK, 0, 0)
        res[name] = {"ms": round(ms, 4), "TOPS": round(t, 1), "frac": round(t / PEAK_INT8_TOPS, 4),
                     "tile": tiles.get(tile, str(tile))}
        if tile != _lib.PATH_MFMA_256x256:  # the 256x256 tile on the same shape, for comparison
            ms2 = timed(lambda: L.fke_qgemm_i8_on_path(_lib.PATH_MFMA_256x256, A.data_ptr(), B.data_ptr(),
                                                       C.data_ptr(), M, N, K, sa.data_ptr(), sb.data_ptr(), 1.0,
                                                       1.0, None, out, _lib.B_NK, sh), args.steps, args.warmup, args.preheat_ms)
            res[name]["ms_256x256_tile"] = round(ms2, 4)
        del A, B, C
    return res


# Shapes around the MFMA tile rule (B [N,K]): 256x256 tiles / 128x128 tiles.
TILE_SWEEP_SHAPES = [
    (256, 4096, 4096), (512, 4096, 4096), (1024, 4096, 4096), (2048, 4096, 4096),  # 16..128 / 64..512
    (3072, 4096, 4096), (4096, 4096, 4096),                                          # 192 / 768, 256 / 1024
    (4096, 512, 4096), (2048, 1376, 4096), (4096, 1376, 4096), (4096, 2048, 4096),   # 32..128 / 128..512
    (4096, 3584, 4096), (512, 14336, 4096), (1024, 14336, 4096),                     # 224 / 896, 112 / 448, 224
    (8192, 1024, 8192), (8192, 8192, 1024), (4096, 11008, 4096),                     # 128 / 512, 1024, 688
    (8192, 8192, 512), (8192, 8192, 2048), (4096, 4096, 1024), (4096, 4096, 2048),   # short K, many tiles
    (4096, 11008, 1024), (4096, 11008, 2048), (16384, 8192, 1024)]


def tile_sweep(torch, L, _lib, dev, gen, timed, args):
    """Every MFMA tile pinned (the FKE_PATH_MFMA_* paths of TILE_LABELS) on each shape, INT8 and FP8
    with bf16 out and bf16 operands with bf16 out, beside the tile fke_select_mfma_tile picks: "warm" reuses
    one weight buffer (it stays in the caches), "cold" cycles the weights over at least 512 MiB of buffers
    (as a model's forward pass meets them).  Each variant runs 30 ms back to back before its timed launches."""
    sh = torch.cuda.current_stream(dev).cuda_stream
    names = TILE_LABELS
    res = {}
    for (M, N, K) in TILE_SWEEP_SHAPES:
        C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        sa = torch.rand(M, device=dev, generator=gen)
        sb = torch.rand(N, device=dev, generator=gen)
        for elem in ("i8", "f8", "bf16"):
            eb = 2 if elem == "bf16" else 1
            nb = max(2, min(64, (512 << 20) // (N * K * eb) + 1))
            if elem == "bf16":
                A = torch.randn((M, K), device=dev, generator=gen).to(torch.bfloat16)
                Bs = [torch.randn((N, K), device=dev, generator=gen).to(torch.bfloat16) for _ in range(nb)]
            else:
                A = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=gen)
                Bs = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=gen) for _ in range(nb)]
                if elem == "f8":  # no NaN codes (those rerun a tile)
                    A[(A & 0x7F) == 0x7F] = 0
                    for B in Bs:
                        B[(B & 0x7F) == 0x7F] = 0
            row = {"pick": names[L.fke_select_mfma_tile(M, N, K, _lib.B_NK, 0, 0)], "cold_buffers": nb}
            for path, name in names.items():
                for mode in ("warm", "cold"):
                    it = [0]

                    def fn():
                        B = Bs[0] if mode == "warm" else Bs[it[0] % nb]
                        it[0] += 1
                        if elem == "i8":
                            return L.fke_qgemm_i8_on_path(path, A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K,
                                                          sa.data_ptr(), sb.data_ptr(), 1.0, 1.0, None, _lib.OUT_BF16,
                                                          _lib.B_NK, sh)
                        if elem == "f8":
                            return L.fke_qgemm_f8_on_path(path, A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K,
                                                          0.01, 0.01, None, _lib.OUT_BF16, _lib.B_NK, sh)
                        return L.fke_gemm_half_on_path(path, A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K,
                                                       _lib.IN_BF16, sa.data_ptr(), sb.data_ptr(), 1.0, 1.0, None,
                                                       _lib.OUT_BF16, _lib.B_NK, sh)
                    if fn() != 0:
                        raise RuntimeError(f"tile sweep: {elem} {name} {M}x{N}x{K} rejected")
                    row[f"us_{name}_{mode}"] = round(timed(fn, 20, 5, preheat_ms=30.0) * 1e3, 2)
            res[f"{elem}_{M}x{N}x{K}_bf16"] = row
            del A, Bs
        del C
    return res


def batch_configs(torch, L, _lib, dev, gen, args):
    """Batched decode on the decode weights (N = 14336, K = 4096): 32, 64, 128 and 256 rows with B [N,K],
    32, 64 and 128 rows with B [K,N] (the reference's layout), and 64 and 128 rows on the LDS-streamed kernel
    pinned. The dispatcher gives 32 rows to the streamed kernel ([K,N]: the split decode) and the larger
    batches to the MFMA GEMM's ring tiles (one tile per CU); each line names its kernel."""
    res = {f"gemv_M{m}": gemv_bench(torch, L, _lib, dev, gen, m, args.gemv_buffers, args.gemv_launches)
           for m in (32, 64, 128, 256)}
    for m in (32, 64, 128):
        res[f"gemv_M{m}_b_kn"] = gemv_bench(torch, L, _lib, dev, gen, m, args.gemv_buffers, args.gemv_launches,
                                            layout="kn")
    for m in (64, 128):  # the streamed decode kernel pinned, for the choice between it and the ring tiles
        res[f"gemv_M{m}_streamed"] = gemv_bench(torch, L, _lib, dev, gen, m, args.gemv_buffers, args.gemv_launches,
                                                path=_lib.PATH_GEMV)
    return res


KSPLIT_SHAPES = [(64, 4096, 14336, "nk"), (128, 8192, 28672, "nk"), (100, 1000, 14720, "nk"),
                 (128, 1024, 8192, "nk"), (300, 528, 8192, "nk"), (200, 2000, 8192, "kn")]


def ksplit_configs(torch, L, _lib, dev, gen, args):
    """The MFMA GEMM's K split (few output tiles, a long K): the dispatcher's call, which splits K, beside
    the unsplit tile the tile rule picks, pinned; cold weights cycled from a HIP graph like the decode
    lines (the byte counts are the operands' and the output's, not the partial sums')."""
    import ctypes
    res = {}
    names = {_lib.PATH_MFMA_64x64_RING4: "64x64_ring4", _lib.PATH_MFMA_128x64_RING4: "128x64_ring4",
             _lib.PATH_MFMA_128x128_RING4: "128x128_ring4", _lib.PATH_MFMA_128x128: "128x128",
             _lib.PATH_MFMA_256x256: "256x256"}
    for M, N, K, lay in KSPLIT_SHAPES:
        code = _lib.B_KN if lay == "kn" else _lib.B_NK
        t = ctypes.c_int(0)
        S = L.fke_select_mfma_split(M, N, K, code, 0, ctypes.byref(t))
        unsplit = L.fke_select_mfma_tile(M, N, K, code, 0, 0)
        nbuf = min(128, max(args.gemv_buffers, -(-(448 << 20) // (N * K))))  # >= 448 MiB of weights: past the MALL
        key = f"ksplit_{M}x{N}x{K}_{lay}"
        r = gemv_bench(torch, L, _lib, dev, gen, M, nbuf, args.gemv_launches, N=N, K=K, layout=lay)
        r["kernel"] = (f"gemm_mfma_kernel {names[t.value]}, {S} K splits + splitk_reduce_kernel" if S > 1
                       else f"{r['kernel']} (unsplit)")
        res[key] = r
        u = gemv_bench(torch, L, _lib, dev, gen, M, nbuf, args.gemv_launches, N=N, K=K, layout=lay, path=unsplit)
        u["kernel"] = f"gemm_mfma_kernel {names[unsplit]} (unsplit, pinned)"
        res[key + "_unsplit"] = u
    return res


def extra_configs(torch, L, _lib, dev, gen, timed, rand_i8, rand_u, args):
    res = {}
    # prefill 4096 x 11008 x 4096, bf16 out
    M, N, K = 4096, 11008, 4096
    A, B, sa, sb = rand_i8(M, K), rand_i8(N, K), rand_u(M), rand_u(N)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    sh = torch.cuda.current_stream(dev).cuda_stream
    ms = timed(lambda: L.fke_qgemm_i8(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, sa.data_ptr(),
                                      sb.data_ptr(), 1.0, 1.0, None, _lib.OUT_BF16, _lib.B_NK, sh),
               args.steps, args.warmup, args.preheat_ms)
    t = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    res["prefill_4096x11008x4096_bf16"] = {"ms": round(ms, 4), "TOPS": round(t, 1),
                                           "frac": round(t / PEAK_INT8_TOPS, 4)}
    del A, B, C
    # INT8 8192^3 with B [K,N] (the layout of the reference's Python op), fp32 out
    M = N = K = 8192
    A, B, sa, sb = rand_i8(M, K), rand_i8(K, N), rand_u(M), rand_u(N)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    ms = timed(lambda: L.fke_qgemm_i8(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, sa.data_ptr(),
                                      sb.data_ptr(), 1.0, 1.0, None, _lib.OUT_F32, _lib.B_KN, sh),
               args.steps, args.warmup, args.preheat_ms)
    t = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    res["int8_8192cubed_f32_Bkn"] = {"ms": round(ms, 4), "TOPS": round(t, 1), "frac": round(t / PEAK_INT8_TOPS, 4)}
    del A, B, C
    res.update(fp8_configs(torch, L, _lib, dev, gen, timed, args))
    # FP8 with 1 in 97 codes of A set to 0x7F: tiles rerun with NaN codes cleared
    M = N = K = 8192
    A8 = torch.randint(0, 256, (M, K), dtype=torch.uint8, device=dev, generator=gen)
    A8[(A8 & 0x7F) == 0x7F] = 0
    B8 = torch.randint(0, 256, (K, N), dtype=torch.uint8, device=dev, generator=gen)
    B8[(B8 & 0x7F) == 0x7F] = 0
    A8.view(-1)[::97] = 0x7F
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ms = timed(lambda: L.fke_qgemm_f8(A8.data_ptr(), B8.data_ptr(), C.data_ptr(), M, N, K, 0.01, 0.01,
                                      None, _lib.OUT_BF16, _lib.B_NK, sh), args.steps, args.warmup, args.preheat_ms)
    t = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    res["fp8_8192cubed_bf16_Bnk_nan_codes"] = {"ms": round(ms, 4), "TFLOPS": round(t, 1),
                                               "frac": round(t / PEAK_FP8_TFLOPS, 4)}
    del A8, B8, C
    res.update(half_configs(torch, L, _lib, dev, gen, timed, args))
    res.update(shard_configs(torch, L, _lib, dev, gen, timed, rand_i8, rand_u, args))
    res["gemv_M4"] = gemv_bench(torch, L, _lib, dev, gen, 4, args.gemv_buffers, args.gemv_launches)
    res.update(batch_configs(torch, L, _lib, dev, gen, args))
    res.update(ksplit_configs(torch, L, _lib, dev, gen, args))
    # per-token INT8 quantiser in front of the W8A8 GEMM: bf16 activations of C3 (4096 x 4096),
    # 12 rotating inputs (384 MiB, more than the MALL), timed from a HIP graph like the GEMV
    M, K, nx = 4096, 4096, 12
    Xs = [torch.randn((M, K), device=dev, generator=gen).to(torch.bfloat16) for _ in range(nx)]
    Q = torch.empty((M, K), dtype=torch.int8, device=dev)
    S = torch.empty(M, dtype=torch.float32, device=dev)

    def qlaunch(i, st):
        r = L.fke_quantize_rows_i8(Xs[i % nx].data_ptr(), _lib.IN_BF16, M, K, Q.data_ptr(), S.data_ptr(), st)
        if r:
            raise RuntimeError(f"quantiser failed: {_lib.status_string(r)}")

    us = graph_us(torch, dev, qlaunch, 240, 2 * nx)
    nbytes = M * K * 2 + M * K + 4 * M
    gbs = nbytes / (us * 1e-6) / 1e9
    res["quantize_rows_4096x4096_bf16"] = {"us": round(us, 2), "GB/s": round(gbs, 1),
                                           "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes,
                                           "kernel": "quant_rows_kernel<bf16>"}
    del Xs, Q, S
    res.update(swiglu_configs(torch, L, _lib, dev, gen, timed, rand_i8, rand_u, args))
    res.update(odd_k_configs(torch, L, _lib, dev, timed, rand_i8, rand_u, args))
    return res


def odd_k_configs(torch, L, _lib, dev, timed, rand_i8, rand_u, args):
    """Prefill W8A8 shapes whose K is not a multiple of the 128-byte stage (bf16
    out, per-token x per-channel scales): the dispatcher's MFMA GEMM (its last
    stage cleared past K; for K % 16 != 0 the word kernel) and the any-shape
    generic kernel pinned on the same call, each with its roofline."""
    res = {}
    sh = torch.cuda.current_stream(dev).cuda_stream
    for M, N, K in ((4096, 11008, 4160), (4096, 4096, 2880), (4096, 11008, 4100)):
        A, B, sa, sb = rand_i8(M, K), rand_i8(N, K), rand_u(M), rand_u(N)
        C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        fast = "words" if K % 16 else "mfma"
        for name, path in ((fast, _lib.PATH_AUTO), ("generic", _lib.PATH_GENERIC)):
            if path == _lib.PATH_AUTO:
                assert L.fke_select_path_i8(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, _lib.OUT_BF16,
                                            _lib.B_NK) == _lib.PATH_MFMA

            def run(path=path):
                st = L.fke_qgemm_i8_on_path(path, A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, sa.data_ptr(),
                                            sb.data_ptr(), 1.0, 1.0, None, _lib.OUT_BF16, _lib.B_NK, sh)
                if st:
                    raise RuntimeError(f"fke_qgemm_i8_on_path failed: {_lib.status_string(st)}")

            steps = args.steps if name != "generic" else max(3, args.steps // 10)
            ms = timed(run, steps, 2 if name == "generic" else args.warmup, args.preheat_ms if name != "generic" else 0)
            t = 2.0 * M * N * K / (ms * 1e-3) / 1e12
            res[f"prefill_{M}x{N}x{K}_bf16_{name}"] = {
                "ms": round(ms, 4), "TOPS": round(t, 1), "frac": round(t / PEAK_INT8_TOPS, 4),
                "kernel": {"mfma": "gemm_mfma_kernel<i8,NK,bf16> (partial last stage)",
                           "words": "gemm_words_kernel<i8,NK,bf16> (4-byte LDS-DMA copies, K % 4 == 0)",
                           "generic": "gemm_generic_kernel<i8>"}[name]}
        del A, B, C
    return res


def data_sweep(torch, L, _lib, dev, gen, timed, args):
    """The headline INT8 GEMM (8192^3, fp32 out, scalar scales) on all-zero, all-one,
    uniform [-3,3] and uniform [-127,127] operands, in that order: the same
    instructions on data of different switching activity, to show the power-limited
    clock (pair with rocprofv3 --pmc GRBM_GUI_ACTIVE for the cycle counts)."""
    res = {}
    sh = torch.cuda.current_stream(dev).cuda_stream
    M = N = K = 8192
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    kinds = (("zeros", None), ("ones", None), ("uniform_-3_3", 3), ("uniform_-127_127", 127))
    for name, r in kinds:
        if r is None:
            fill = 0 if name == "zeros" else 1
            A = torch.full((M, K), fill, dtype=torch.int8, device=dev)
            B = torch.full((N, K), fill, dtype=torch.int8, device=dev)
        else:
            A = torch.randint(-r, r + 1, (M, K), dtype=torch.int8, device=dev, generator=gen)
            B = torch.randint(-r, r + 1, (N, K), dtype=torch.int8, device=dev, generator=gen)
        ms = timed(lambda: L.fke_qgemm_i8(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, None, None, 1.0, 1.0,
                                          None, _lib.OUT_F32, _lib.B_NK, sh), args.steps, args.warmup, args.preheat_ms)
        res[name] = {"ms": round(ms, 4), "TOPS": round(2.0 * M * N * K / ms / 1e9, 1)}
        del A, B
    return res


def mfma_ceiling(torch, dev, gen, timed, args):
    """What the matrix cores sustain on their own, at the board's power limit:
    one workgroup of 4 waves per CU streams v_mfma_i32_32x32x32_i8 in the
    GEMM's 4x4-block order on operands held in registers (no LDS, no memory
    traffic in the loop; csrc/probe_mfma.hip), for operands drawn as the
    headline's (uniform int8 [-127,127]) and for constant ones.  Each runs
    back to back for the pre-heat time, then `steps` timed launches, then
    1.1 s more while amdsmi reads the clock and socket power."""
    import ctypes as ct
    P = ct.CDLL(os.path.join(PKG, "lib", "libfke_probe.so"))
    P.fke_probe_mfma_src_bytes.argtypes = [ct.c_int]
    P.fke_probe_mfma_src_bytes.restype = ct.c_size_t
    P.fke_probe_mfma_out_elems.argtypes = [ct.c_int]
    P.fke_probe_mfma_out_elems.restype = ct.c_size_t
    P.fke_probe_mfma_i8.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_int, ct.c_void_p]
    P.fke_probe_mfma_i8.restype = ct.c_int
    sh = torch.cuda.current_stream(dev).cuda_stream
    grid = torch.cuda.get_device_properties(dev).multi_processor_count
    iters = 2048
    out = torch.empty(P.fke_probe_mfma_out_elems(grid), dtype=torch.int32, device=dev)
    nbytes = P.fke_probe_mfma_src_bytes(grid)
    ops = float(grid) * 4 * iters * 32 * 2 * 32 * 32 * 32
    res = {"grid": grid, "iters": iters, "ops_per_launch": ops}
    for name, src in (("uniform_-127_127", torch.randint(-127, 128, (nbytes,), dtype=torch.int8, device=dev,
                                                           generator=gen)),
                      ("ones", torch.ones(nbytes, dtype=torch.int8, device=dev))):
        def fn():
            st = P.fke_probe_mfma_i8(src.data_ptr(), out.data_ptr(), grid, iters, sh)
            if st:
                raise RuntimeError(f"fke_probe_mfma_i8 failed: status {st}")
        torch.cuda.synchronize()
        clock = ClockSampler() if args.clock_ms > 0 else None
        if clock:
            clock.start()
        ms = timed(fn, max(args.steps, 20), 5, args.preheat_ms)
        if clock:
            preheat(torch, fn, args.clock_ms)
        sclk = clock.stop() if clock else None
        pops = ops / (ms * 1e-3) / 1e15
        res[name] = {"ms": round(ms, 4), "POPs": round(pops, 3), "frac_of_peak": round(pops * 1e3 / PEAK_INT8_TOPS, 4),
                     "sclk_mhz": sclk}
        del src
    return res


def fp8_configs(torch, L, _lib, dev, gen, timed, args):
    """FP8 e4m3 8192^3, B [K,N] (reference layout) and [N,K], bf16 out; FP8 decode M=1,16."""
    res = {}
    sh = torch.cuda.current_stream(dev).cuda_stream
    M = N = K = 8192
    A8 = torch.randint(0, 256, (M, K), dtype=torch.uint8, device=dev, generator=gen)
    A8[(A8 & 0x7F) == 0x7F] = 0
    B8 = torch.randint(0, 256, (K, N), dtype=torch.uint8, device=dev, generator=gen)
    B8[(B8 & 0x7F) == 0x7F] = 0
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    for name, lay in (("kn", _lib.B_KN), ("nk", _lib.B_NK)):
        ms = timed(lambda: L.fke_qgemm_f8(A8.data_ptr(), B8.data_ptr(), C.data_ptr(), M, N, K, 0.01, 0.01,
                                          None, _lib.OUT_BF16, lay, sh), args.steps, args.warmup, args.preheat_ms)
        t = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        res[f"fp8_8192cubed_bf16_B{name}"] = {"ms": round(ms, 4), "TFLOPS": round(t, 1),
                                              "frac": round(t / PEAK_FP8_TFLOPS, 4)}
    del A8, B8, C
    # FP8 decode on the decode weights (N = 14336, K = 4096, B [N,K], bf16 out + bias): the
    # row kernel at M = 1 and the LDS-streamed kernel at M = 16, 8 rotating weights, HIP-graph
    # timed like the INT8 decode lines
    N, K, nbuf = 14336, 4096, args.gemv_buffers
    Bs = []
    for _ in range(nbuf):
        b = torch.randint(0, 256, (N, K), dtype=torch.uint8, device=dev, generator=gen)
        b[(b & 0x7F) == 0x7F] = 0
        Bs.append(b)
    bias = torch.randn(N, device=dev, generator=gen) * 0.02
    # the same bytes read as B [K,N] (the reference launcher's layout) run the transposing decode kernel
    for lname, lay in (("", _lib.B_NK), ("_Bkn", _lib.B_KN)):
        for M in (1, 16):
            if lay == _lib.B_KN:
                kern = ("gemv_kn_row_kernel<f8>" if M == 1 else "gemv_kn_split_kernel<f8>") + "+kn_reduce_kernel<f8>"
            else:
                kern = "gemv_rows_kernel (FP8)" if M == 1 else "gemv_lds_kernel (FP8)"
            A8 = torch.randint(0, 256, (M, K), dtype=torch.uint8, device=dev, generator=gen)
            A8[(A8 & 0x7F) == 0x7F] = 0
            out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

            def launch(i, st):
                r = L.fke_qgemm_f8(A8.data_ptr(), Bs[i % nbuf].data_ptr(), out.data_ptr(), M, N, K, 0.01, 0.01,
                                   bias.data_ptr(), _lib.OUT_BF16, lay, st)
                if r:
                    raise RuntimeError(f"fp8 decode failed: {_lib.status_string(r)}")

            us = graph_us(torch, dev, launch, args.gemv_launches, 2 * nbuf)
            nbytes = M * K + N * K + 4 * N + 2 * M * N
            gbs = nbytes / (us * 1e-6) / 1e9
            res[f"fp8_decode_M{M}_14336x4096_bf16{lname}"] = {"us": round(us, 3), "GB/s": round(gbs, 1),
                                                              "frac": round(gbs / PEAK_HBM_GBS, 4),
                                                              "bytes": nbytes, "kernel": kern}
    del Bs
    return res


def vendor_configs(torch, dev, gen, timed, args):
    """The vendor library (hipBLASLt through torch) on the 8192^3 GEMMs, timed like
    this library's: INT8 (torch._int_mm, int32 out), FP8 e4m3 (torch._scaled_mm,
    bf16 out), bf16 and fp16 (A @ B^T, same-type out).  Context only, not a bench figure."""
    res = {}
    M = N = K = 8192
    A = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=gen)
    B = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=gen)
    ms = timed(lambda: torch._int_mm(A, B.t()), args.steps, args.warmup, args.preheat_ms)
    res["int8_8192cubed_i32out_torch_int_mm"] = {"ms": round(ms, 4), "TOPS": round(2.0 * M * N * K / ms / 1e9, 1)}
    del A, B
    try:
        a8 = torch.randn((M, K), device=dev, generator=gen).to(torch.float8_e4m3fn)
        b8 = torch.randn((N, K), device=dev, generator=gen).to(torch.float8_e4m3fn)
        one = torch.tensor(1.0, device=dev)
        ms = timed(lambda: torch._scaled_mm(a8, b8.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16),
                   args.steps, args.warmup, args.preheat_ms)
        res["fp8_8192cubed_bf16out_torch_scaled_mm"] = {"ms": round(ms, 4),
                                                       "TFLOPS": round(2.0 * M * N * K / ms / 1e9, 1)}
        del a8, b8
    except (RuntimeError, AttributeError) as e:  # the op may be absent for this device / build
        res["fp8_8192cubed_bf16out_torch_scaled_mm"] = {"error": str(e)[:200]}
    for name, dt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        Ah = torch.randn((M, K), device=dev, generator=gen).to(dt)
        Bh = torch.randn((N, K), device=dev, generator=gen).to(dt)
        ms = timed(lambda: Ah @ Bh.t(), args.steps, args.warmup, args.preheat_ms)
        res[f"{name}_8192cubed_torch_matmul"] = {"ms": round(ms, 4), "TFLOPS": round(2.0 * M * N * K / ms / 1e9, 1)}
        del Ah, Bh
    return res


def half_configs(torch, L, _lib, dev, gen, timed, args):
    """fp16 / bf16 GEMM 8192^3 on the MFMA engine (B [N,K], bf16 out)."""
    res = {}
    sh = torch.cuda.current_stream(dev).cuda_stream
    M = N = K = 8192
    for name, dt, code in (("bf16", torch.bfloat16, _lib.IN_BF16), ("f16", torch.float16, _lib.IN_F16)):
        Ah = torch.randn((M, K), device=dev, generator=gen).to(dt)
        Bh = torch.randn((N, K), device=dev, generator=gen).to(dt)
        C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        ms = timed(lambda: L.fke_gemm_half(Ah.data_ptr(), Bh.data_ptr(), C.data_ptr(), M, N, K, code, None, None,
                                           1.0, 1.0, None, _lib.OUT_BF16, _lib.B_NK, sh), args.steps, args.warmup, args.preheat_ms)
        t = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        res[f"{name}_gemm_8192cubed_bf16out"] = {"ms": round(ms, 4), "TFLOPS": round(t, 1),
                                                 "frac": round(t / PEAK_BF16_TFLOPS, 4),
                                                 "kernel": f"gemm_mfma_kernel<{name}, nk, bf16>"}
        del Ah, Bh, C
    return res


def swiglu_configs(torch, L, _lib, dev, gen, timed, rand_i8, rand_u, args):
    """The MLP gate/up projection of a Llama-3-8B-shaped layer (K = 4096,
    I = 14336) with SwiGLU fused into the GEMM epilogue, against the unfused
    pipeline (two GEMMs to bf16, then the elementwise op), plus the elementwise
    op alone and the decode (M = 1) fused kernel."""
    res = {}
    sh = torch.cuda.current_stream(dev).cuda_stream
    M, I, K = 4096, 14336, 4096
    A, W, sa, sb = rand_i8(M, K), rand_i8(2 * I, K), rand_u(M), rand_u(2 * I)
    H = torch.empty((M, I), dtype=torch.bfloat16, device=dev)
    G = torch.empty((M, I), dtype=torch.bfloat16, device=dev)
    U = torch.empty((M, I), dtype=torch.bfloat16, device=dev)
    ms = timed(lambda: L.fke_qgemm_i8_swiglu(A.data_ptr(), W.data_ptr(), H.data_ptr(), M, I, K, sa.data_ptr(),
                                             sb.data_ptr(), 1.0, 1.0, None, _lib.OUT_BF16, sh),
               args.steps, args.warmup, args.preheat_ms)
    Wu = W[I:]
    sbu = sb[I:]

    def unfused():
        L.fke_qgemm_i8(A.data_ptr(), W.data_ptr(), G.data_ptr(), M, I, K, sa.data_ptr(), sb.data_ptr(), 1.0, 1.0,
                       None, _lib.OUT_BF16, _lib.B_NK, sh)
        L.fke_qgemm_i8(A.data_ptr(), Wu.data_ptr(), U.data_ptr(), M, I, K, sa.data_ptr(), sbu.data_ptr(), 1.0,
                       1.0, None, _lib.OUT_BF16, _lib.B_NK, sh)
        L.fke_swiglu(G.data_ptr(), U.data_ptr(), H.data_ptr(), M * I, _lib.IN_BF16, sh)

    ms_u = timed(unfused, args.steps, args.warmup, args.preheat_ms)
    t = 2.0 * M * 2 * I * K / (ms * 1e-3) / 1e12
    res["swiglu_gate_up_4096x14336x4096_bf16"] = {
        "ms": round(ms, 4), "TOPS": round(t, 1), "frac": round(t / PEAK_INT8_TOPS, 4),
        "unfused_ms": round(ms_u, 4), "speedup_vs_unfused": round(ms_u / ms, 3),
        "kernel": "gemm_mfma_kernel<i8, nk, bf16, swiglu>",
        "unfused": "two gemm_mfma_kernel launches to bf16 [4096,14336] + swiglu_kernel<bf16>"}
    # the elementwise op alone on those bf16 tensors, two rotating sets (704 MiB)
    G2, U2, H2 = torch.empty_like(G), torch.empty_like(U), torch.empty_like(H)
    G.copy_(torch.randn((M, I), device=dev, generator=gen))
    U.copy_(torch.randn((M, I), device=dev, generator=gen))
    G2.copy_(G)
    U2.copy_(U)
    sets = [(G, U, H), (G2, U2, H2)]

    def elaunch(i, st):
        g, u, h = sets[i % 2]
        r = L.fke_swiglu(g.data_ptr(), u.data_ptr(), h.data_ptr(), M * I, _lib.IN_BF16, st)
        if r:
            raise RuntimeError(f"swiglu failed: {_lib.status_string(r)}")

    us = graph_us(torch, dev, elaunch, 40, 4)
    nbytes = 3 * 2 * M * I
    gbs = nbytes / (us * 1e-6) / 1e9
    res["swiglu_elementwise_4096x14336_bf16"] = {"us": round(us, 2), "GB/s": round(gbs, 1),
                                                 "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes,
                                                 "kernel": "swiglu_kernel<bf16, vec>"}
    del A, W, H, G, U, G2, U2, H2, sets
    # decode: M = 1 and 16, fused gate/up + SwiGLU, 4 rotating weights of 112 MiB (448 MiB)
    nbuf = 4
    Ws = [torch.randint(-127, 128, (2 * I, K), dtype=torch.int8, device=dev, generator=gen) for _ in range(nbuf)]
    sb = rand_u(2 * I)
    bias = torch.randn(2 * I, device=dev, generator=gen) * 0.02
    for M in (1, 16):
        A = torch.clamp(torch.round(torch.randn((M, K), device=dev, generator=gen) * 30), -127, 127).to(torch.int8)
        sa = rand_u(M)
        H = torch.empty((M, I), dtype=torch.bfloat16, device=dev)

        def dlaunch(i, st):
            r = L.fke_qgemm_i8_swiglu(A.data_ptr(), Ws[i % nbuf].data_ptr(), H.data_ptr(), M, I, K, sa.data_ptr(),
                                      sb.data_ptr(), 1.0, 1.0, bias.data_ptr(), _lib.OUT_BF16, st)
            if r:
                raise RuntimeError(f"swiglu decode failed: {_lib.status_string(r)}")

        us = graph_us(torch, dev, dlaunch, 200, 2 * nbuf)
        nbytes = M * K + 2 * I * K + 4 * M + 8 * 2 * I + 2 * M * I
        gbs = nbytes / (us * 1e-6) / 1e9
        res[f"swiglu_gate_up_decode_M{M}_14336x4096_bf16"] = {
            "us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes,
            "kernel": "gemv_rows_kernel<1, bf16, fullk, swiglu>" if M <= 2 else "gemv_lds_kernel<bf16, swiglu>"}
        del A, H
    del Ws
    return res


def cpu_baseline(seconds):
    """The reference's host GEMM loop (tests/test_quantized_gemm.cu:39-48, restated
    in oracle/fke_oracle.c), one thread, on a row sample of the 8192^3 problem."""
    import numpy as np

    from oracle import oracle as o
    o.build()
    K = N = 8192
    B = o.gen_i8_uniform((N, K), 2)
    A = o.gen_i8_uniform((1024, K), 1)
    # calibrate on 2 rows, then run a sample sized to about `seconds`
    t0 = time.perf_counter()
    o.ref_host_gemm_i8(A[:2], B, 0.01, 0.02)
    per_row = (time.perf_counter() - t0) / 2
    rows = int(max(2, min(1024, seconds / max(per_row, 1e-6))))
    t0 = time.perf_counter()
    o.ref_host_gemm_i8(A[:rows], B, 0.01, 0.02)
    dt = time.perf_counter() - t0
    tops = 2.0 * rows * N * K / dt / 1e12
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    # the same int32 loop split over rows with OpenMP on the cores the box grants (16 per GPU here)
    nth = min(16, os.cpu_count() or 1)
    arows = max(nth, min(1024, int(4.0 * nth / max(per_row, 1e-6))))
    t0 = time.perf_counter()
    o.w8a8_acc(A[:arows], B, nthreads=nth)
    adt = time.perf_counter() - t0
    all_tops = 2.0 * arows * N * K / adt / 1e12
    return {"value": round(tops, 6), "unit": "TOPS", "cores": 1, "kind": "port",
            "sample": f"{rows} rows x 8192 x 8192 of the 8192^3 INT8 GEMM ({dt:.1f} s), "
                      f"reference host loop restated in C, g++/gcc -O3, 1 thread",
            "all_cores": {"value": round(all_tops, 6), "unit": "TOPS", "cores": nth,
                          "sample": f"{arows} rows x 8192 x 8192 ({adt:.1f} s), the same int32 loop, "
                                    f"OpenMP over rows"},
            "host_cpu": cpu, "host_nproc": os.cpu_count(),
            "gpu_over_cpu_note": "reported baseline, not the target"}


if __name__ == "__main__":
    main()
