"""Benchmark of the gfx950 W4A4 ConvRot linear path.

One step = the four quantized linears of a Flux-class DiT block at M = 4608
tokens (4096 image + 512 text at 1024^2), each run as on the forward path of
the Linear replacement: fused rotate+int4-quantize of the bf16 activation
(written in the bf6 operand layout), then the W4A4 GEMM on the bf6 matrix
cores (exact integer accumulation) with the dequant + bias epilogue to bf16.
``--path int8`` times the packed-int4 / int8-MFMA kernels instead.

    qkv      3072 -> 9216      proj     3072 -> 3072
    mlp_up   3072 -> 12288     mlp_down 12288 -> 3072

Inputs are synthetic and resident in HBM before timing: x ~ N(0,1) with 1% of
channels x20, W ~ N(0, 0.02) in fp16 quantized once by the same kernel and
re-encoded for the bf6 GEMM (load time, untimed), bias ~ N(0, 0.01).  Every linear has its own activation buffer
(~450 MB live per step, beyond the 256 MB Infinity Cache).

Prints one JSON line: value = effective W4A4 linear TOPS of the whole step
(2*M*N*K summed over the four linears / step time, rotate+quant included).
"""
from __future__ import annotations

import argparse
import ctypes
import importlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))

METRIC = "W4A4 linear TOPS (%int8 MFMA peak) + rotate-quant GB/s at M=4608,K=3072"
PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA
PEAK_FP6_TFLOPS = 10100.0    # MI355X dense fp6 / fp4 MFMA (the bf6 GEMM's instruction)
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
M_TOKENS = 4608
G = 256
LINEARS = [("qkv", 3072, 9216), ("proj", 3072, 3072), ("mlp_up", 3072, 12288), ("mlp_down", 12288, 3072)]


TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "w4a4_gemm_bf6_flux_m4608_traffic.md")


class HipTimer:
    """A row of HIP events on one stream, created with hipEventReleaseToDevice
    (a device-scope release when recorded, not the default system-scope one,
    so recording an event does not write the L2 back).  Recorded once after
    every launch, the interval between consecutive events is one launch: the
    kernel plus its dispatch (about 2 us at M=4608, which back-to-back
    launches without events hide)."""
    RELEASE_TO_DEVICE = 0x40000000          # hipEventReleaseToDevice (hip_runtime_api.h)

    def __init__(self, n: int, stream_ptr: int):
        hip = ctypes.CDLL("libamdhip64.so.7")   # resolves to the HIP runtime torch has loaded
        hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.hip, self.stream = hip, ctypes.c_void_p(stream_ptr)
        self.ev = []
        for _ in range(n):
            e = ctypes.c_void_p()
            self._check(hip.hipEventCreateWithFlags(ctypes.byref(e), self.RELEASE_TO_DEVICE), "create")
            self.ev.append(e)

    @staticmethod
    def _check(rc, what):
        if rc != 0:
            raise RuntimeError(f"hipEvent{what} failed: hipError {rc}")

    def record(self, i: int):
        self._check(self.hip.hipEventRecord(self.ev[i], self.stream), "Record")

    def seconds(self, i: int, j: int) -> float:
        """Time from event i to event j (both recorded and complete)."""
        ms = ctypes.c_float()
        self._check(self.hip.hipEventElapsedTime(ctypes.byref(ms), self.ev[i], self.ev[j]), "ElapsedTime")
        return ms.value * 1e-3

    def close(self):
        for e in self.ev:
            self.hip.hipEventDestroy(e)
        self.ev = []


def gpu_lead(torch, buf, fills=4):
    """Queue about a millisecond of unrelated GPU work (fills of `buf`, 1 GiB)
    ahead of a timed sequence, so that the host enqueues the sequence's short
    launches and events while the GPU is still busy: the launches then run back
    to back instead of waiting for the host one by one."""
    for _ in range(fills):
        buf.fill_(0)


def clock_ramp(torch, step, seconds):
    """Untimed steps for about `seconds` of wall time (--clock-ramp-ms), before
    the warmup steps the command line asks for.  The GPU leaves its idle clocks only after
    some milliseconds of sustained load: on MI355X, 20 steps timed after 5
    warmup steps (about 2 ms of work) ran 14% slower than after 50, so a short
    warmup alone would time the clock ramp rather than the kernels.  Returns the
    number of steps run (reported in the JSON line)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            step()
        n += 8
        torch.cuda.synchronize()
    return n


def measured_traffic(key="traffic_bytes_per_launch"):
    """HBM bytes per launch as measured by the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs of this workload, scaled by the 1 GiB copy calibration:
    ``traffic_bytes_per_launch`` for the bf6 GEMM (mean over the four linears),
    ``rotquant_traffic_bytes_per_launch`` for the B6T rotate+quant at
    M=4608, K=3072.  None when that summary is absent."""
    try:
        for line in open(TRAFFIC_SUMMARY):
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def rq_bytes(M, K, path="bf6"):
    """Algorithmic HBM bytes of one rotate+quant launch: read bf16, write the codes
    (bf6 layout: 0.75 B per element over rows padded to 256; int4: 0.5 B; the W8A8
    tier's int8: 1 B) + scales."""
    if path == "bf6":
        codes = ((M + 255) // 256 * 256) * K * 3 // 4
    elif path == "w8a8":
        codes = M * K
    else:
        codes = M * K // 2
    return M * K * 2 + codes + 4 * M


class Linear:
    def __init__(self, torch, native, name, K, N, seed):
        from inputs import normal_bias, normal_weight, outlier_activations
        dev = torch.device("cuda")
        self.name, self.K, self.N, self.M = name, K, N, M_TOKENS
        self.x = outlier_activations(M_TOKENS, K, seed=seed).to(dev)
        w = normal_weight(N, K, seed=seed + 1).to(dev)
        self.qw, self.ws = native.convrot_quant_int4(w, G)         # load-time weight quantization
        self.w6 = native.int4_to_bf6(self.qw)                        # load-time bf6 operand encoding
        self.qw8, self.ws8 = native.convrot_quant_int8(w, G)       # the int8 tier's weight
        self.w8t = native.int8_to_i8t(self.qw8)                      # load-time I8T operand layout
        self.q8 = torch.empty((native.i8t_rows(M_TOKENS), K), dtype=torch.int8, device=dev)
        self.bias = normal_bias(N, seed=seed + 2).to(dev).float()
        self.qx = torch.empty((M_TOKENS, K // 2), dtype=torch.int8, device=dev)
        self.a6 = torch.empty((native.bf6_rows(M_TOKENS), K // 4 * 3), dtype=torch.uint8, device=dev)
        self.xs = torch.empty((M_TOKENS,), dtype=torch.float32, device=dev)
        self.out = torch.empty((M_TOKENS, N), dtype=torch.bfloat16, device=dev)
        del w

    def ops(self):
        return 2.0 * self.M * self.N * self.K


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # 50 untimed steps (about 25 ms of load on the block linears) bring the GPU
    # to steady clocks: after 5, the next 20 steps still ran 14% slower
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--clock-ramp-ms", type=float, default=30.0,
                    help="untimed steps for this long before the warmup steps (0: none)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="approximate CPU time for the oracle baseline (0 disables it)")
    ap.add_argument("--path", choices=("bf6", "int8", "w8a8"), default="bf6",
                    help="GEMM path: bf6 matrix cores (the Linear's), packed int4 on int8 MFMA, or the "
                         "W8A8 tier (int8 activations and weights on int8 MFMA)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 1 GiB device copy (counter calibration)")
    ap.add_argument("--workload", choices=("block-linears", "dit8", "gemm-sweep", "rotquant"),
                    default="block-linears",
                    help="block-linears: the four linears of one DiT block (the headline line); "
                         "dit8: the synthetic 8-block double-stream DiT stack through Int4ConvRotOps; "
                         "gemm-sweep: the W4A4 GEMM alone over a token sweep (k-split as the Linear chooses); "
                         "rotquant: the fused rotate+quantize kernel alone at M=4608 and M=16384")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (every box here has one); --gpus {args.gpus} "
              "is not supported", file=sys.stderr)
        sys.exit(2)
    if args.workload == "dit8":
        bench_dit(args)
        return
    if args.workload == "gemm-sweep":
        bench_gemm_sweep(args)
        return
    if args.workload == "rotquant":
        bench_rotquant(args)
        return

    import torch
    importlib.import_module("comfyui-int4-convrot-rdna4_amd")
    native = importlib.import_module("comfyui-int4-convrot-rdna4_amd._int4.native")
    if not native.is_available():
        raise SystemExit("libconvrot_gfx950.so is not loadable on a gfx950 device; nothing to measure")
    lib = native.load_library()
    stream = torch.cuda.current_stream()
    sptr = ctypes.c_void_p(stream.cuda_stream)

    lins = [Linear(torch, native, n, K, N, seed=10 * i) for i, (n, K, N) in enumerate(LINEARS)]
    torch.cuda.synchronize()

    vp = ctypes.c_void_p
    calls = []   # (kind, index, fn, args)
    for i, L in enumerate(lins):
        if args.path == "bf6":
            calls.append(("rq", i, lib.cr_convrot_quant_bf6,
                          (vp(L.x.data_ptr()), 1, vp(L.a6.data_ptr()), vp(L.xs.data_ptr()), L.M, L.K, G, sptr)))
            calls.append(("gemm", i, lib.cr_int4_convrot_gemm_bf6,
                          (vp(L.a6.data_ptr()), vp(L.w6.data_ptr()), vp(L.xs.data_ptr()), vp(L.ws.data_ptr()),
                           vp(L.bias.data_ptr()), vp(L.out.data_ptr()), L.M, L.N, L.K, 1, sptr)))
        elif args.path == "w8a8":   # the int8 linear's path: I8T operands (K % 64 == 0)
            calls.append(("rq", i, lib.cr_convrot_quant_int8_i8t,
                          (vp(L.x.data_ptr()), 1, vp(L.q8.data_ptr()), vp(L.xs.data_ptr()), L.M, L.K, G, sptr)))
            calls.append(("gemm", i, lib.cr_int8_convrot_gemm_i8t,
                          (vp(L.q8.data_ptr()), vp(L.w8t.data_ptr()), vp(L.xs.data_ptr()), vp(L.ws8.data_ptr()),
                           vp(L.bias.data_ptr()), vp(L.out.data_ptr()), L.M, L.N, L.K, 1, sptr)))
        else:
            calls.append(("rq", i, lib.ck_convrot_quant_int4,
                          (vp(L.x.data_ptr()), 1, vp(L.qx.data_ptr()), vp(L.xs.data_ptr()), L.M, L.K, G, sptr)))
            calls.append(("gemm", i, lib.ck_int4_convrot_gemm,
                          (vp(L.qx.data_ptr()), vp(L.qw.data_ptr()), vp(L.xs.data_ptr()), vp(L.ws.data_ptr()),
                           vp(L.bias.data_ptr()), vp(L.out.data_ptr()), L.M, L.N, L.K, 1, sptr)))

    def step(timer=None, base=0):
        for j, (_, _, fn, a) in enumerate(calls):
            rc = fn(*a)
            if timer is not None:
                timer.record(base + j + 1)
            if rc != 0:
                raise RuntimeError(f"launch failed rc={rc}")

    ramp_steps = clock_ramp(torch, step, args.clock_ramp_ms * 1e-3)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: K steps, bracketed by synchronize on both sides, with no
    # event between the launches (an event record is a packet of its own on the
    # stream and would be timed as part of the step)
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    t_start.record(stream)
    for s in range(args.steps):
        step()
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = t_start.elapsed_time(t_end) / args.steps

    # per-launch durations: the same K steps again with one HIP event on the
    # launch stream after every launch (and one before the first), so launch j
    # is timed from the event before it to the event after it.  Each interval
    # also holds the ~2 us dispatch of its launch that back-to-back launches
    # hide, so these durations sit a little above a kernel trace's.
    nc = len(calls)
    timer = HipTimer(args.steps * nc + 1, stream.cuda_stream)
    torch.cuda.synchronize()
    timer.record(0)
    for s in range(args.steps):
        step(timer, s * nc)
    torch.cuda.synchronize()
    ms_step_events = timer.seconds(0, args.steps * nc) * 1e3 / args.steps
    dur = {}
    for s in range(args.steps):
        for j, (kind, i, _, _) in enumerate(calls):
            dur.setdefault((kind, i), []).append(timer.seconds(s * nc + j, s * nc + j + 1))
    timer.close()
    avg = {k: sum(v) / len(v) for k, v in dur.items()}

    total_ops = sum(L.ops() for L in lins)
    value = total_ops / (ms_step * 1e-3) / 1e12
    gemm_time = sum(avg[("gemm", i)] for i in range(len(lins)))
    gemm_launch_avg = gemm_time / len(lins)
    gemm_ops_avg = total_ops / len(lins)
    gemm_tops = gemm_ops_avg / gemm_launch_avg / 1e12
    rq_time = sum(avg[("rq", i)] for i in range(len(lins)))
    rq_b = sum(rq_bytes(L.M, L.K, args.path) for L in lins)
    rq_gbs = rq_b / rq_time / 1e9
    metric_rq = avg[("rq", 1)]                   # proj input: M=4608, K=3072
    metric_rq_gbs = rq_bytes(M_TOKENS, 3072, "int4") / metric_rq / 1e9

    detail = {}
    for i, L in enumerate(lins):
        detail[L.name] = {
            "K": L.K, "N": L.N,
            "rotate_quant_us": round(avg[("rq", i)] * 1e6, 2),
            "rotate_quant_GBps": round(rq_bytes(L.M, L.K, args.path) / avg[("rq", i)] / 1e9, 1),
            "gemm_us": round(avg[("gemm", i)] * 1e6, 2),
            "gemm_TOPS": round(L.ops() / avg[("gemm", i)] / 1e12, 1),
        }

    # Each linear's GEMM as a burst: back-to-back launches over copies of its
    # weight operand (>= 300 MB in all, beyond the 256 MB Infinity Cache, so
    # each launch reads its weight from HBM, as in the step), on the
    # activation the step's rotate+quant wrote, bracketed by two HIP events
    # with none in between: the average launch duration, without the per-launch
    # event gap of the intervals above.
    gemm_burst = {}
    if args.path == "bf6":
        lead = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        for i, L in enumerate(lins):
            kind, _, gfn, gargs = calls[2 * i + 1]
            assert kind == "gemm"
            ncopy = max(2, (300 << 20) // L.w6.numel() + 1)
            w6s = [L.w6.clone() for _ in range(ncopy)]
            nb = 2 * ncopy

            def gburst():
                for b in range(nb):
                    a = tuple(gargs[:1]) + (vp(w6s[b % ncopy].data_ptr()),) + tuple(gargs[2:])
                    if gfn(*a) != 0:
                        raise RuntimeError("GEMM launch failed")
            gburst()
            bt = HipTimer(2, stream.cuda_stream)
            torch.cuda.synchronize()
            gpu_lead(torch, lead)
            bt.record(0)
            gburst()
            bt.record(1)
            torch.cuda.synchronize()
            gemm_burst[L.name] = bt.seconds(0, 1) / nb
            bt.close()
            del w6s
        del lead

    # The metric-point rotate+quant (M=4608, K=3072) as a burst: back-to-back
    # launches over enough distinct inputs (>= 600 MB, beyond the 256 MB
    # Infinity Cache) that each reads its x from HBM, bracketed by two HIP events
    # on the launch stream and no event in between, so the average launch
    # duration holds no per-launch event gap (the intervals above do: about
    # 2-5 us of dispatch each, which back-to-back launches hide).
    rq_fn, rq_args = calls[2][2], calls[2][3]
    assert calls[2][0] == "rq" and lins[1].K == 3072
    nbuf = (600 << 20) // (M_TOKENS * 3072 * 2) + 1
    xbufs = [lins[1].x.roll(b, 0).contiguous() for b in range(nbuf)]
    burst = 2 * nbuf
    lead = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")

    def rq_burst(timer=None):
        for b in range(burst):
            a = (vp(xbufs[b % nbuf].data_ptr()),) + tuple(rq_args[1:])
            if rq_fn(*a) != 0:
                raise RuntimeError("rotate+quant launch failed")

    rq_burst()
    bt = HipTimer(2, stream.cuda_stream)
    torch.cuda.synchronize()
    gpu_lead(torch, lead)
    bt.record(0)
    rq_burst()
    bt.record(1)
    torch.cuda.synchronize()
    rq_burst_us = bt.seconds(0, 1) / burst * 1e6
    bt.close()
    del xbufs, lead
    rq_alg = rq_bytes(M_TOKENS, 3072, "int4")          # the metric's bytes: bf16 in, packed int4 + scales out
    rq_alg_layout = rq_bytes(M_TOKENS, 3072, args.path)

    copy_cal = None
    if args.copy_calibration:
        a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        copy_cal = {"bytes_read": 1 << 30, "bytes_written": 1 << 30}
        del a, b

    cpu = cpu_baseline_torch(args.cpu_seconds) if args.cpu_seconds > 0 else None
    cpu_c = cpu_baseline(args.cpu_seconds) if args.cpu_seconds > 0 else None

    if gemm_burst:
        # the roofline's launch duration: the burst average (the step's event
        # intervals stay in detail as gemm_us_step_events)
        gemm_launch_avg = sum(gemm_burst.values()) / len(gemm_burst)
        gemm_tops = gemm_ops_avg / gemm_launch_avg / 1e12
        for L in lins:
            d = detail[L.name]
            d["gemm_us_step_events"], d["gemm_TOPS_step_events"] = d["gemm_us"], d["gemm_TOPS"]
            d["gemm_us"] = round(gemm_burst[L.name] * 1e6, 2)
            d["gemm_TOPS"] = round(L.ops() / gemm_burst[L.name] / 1e12, 1)

    line = {
        "metric": METRIC if args.path != "w8a8" else METRIC.replace("W4A4", "W8A8"),
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_ramp_steps": ramp_steps,      # untimed, before the warmup (clock_ramp)
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # the path's arithmetic: int4 codes (int8 codes for the W8A8 tier) with exact
        # integer accumulation; the products run on BF6 / int8 matrix cores
        "dtype": "int8" if args.path == "w8a8" else "int4",
        "data": "synthetic",
        "config": {
            "workload": "Flux-class DiT block W4A4 ConvRot linears (qkv 3072->9216, proj 3072->3072, "
                        "mlp_up 3072->12288, mlp_down 12288->3072), M=4608 tokens, bf16 in/out, G=256",
            "M": M_TOKENS, "convrot_groupsize": G, "linears": [[n, K, N] for n, K, N in LINEARS],
            "gemm_path": args.path,
        },
        "roofline": {
            "kernel": {"bf6": "w4a4_gemm_bf6_kernel<EPI_BF16> (v_mfma_scale_f32_32x32x64_f8f6f4, BF6 operands)",
                       "int8": "w4a4_gemm_pipe_kernel<EPI_BF16> (v_mfma_i32_32x32x32_i8, int4 unpacked)",
                       "w8a8": "w4a4_gemm_pipe_kernel<EPI_BF16, I8, I8T> (v_mfma_i32_32x32x32_i8, int8 operands in the I8T layout)"}[args.path],
            "bound": "mfma",
            "achieved": round(gemm_tops, 1),
            "peak": PEAK_FP6_TFLOPS if args.path == "bf6" else PEAK_INT8_TOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tops / (PEAK_FP6_TFLOPS if args.path == "bf6" else PEAK_INT8_TOPS), 4),
            "traffic": measured_traffic() if args.path == "bf6" else None,
        },
        "rotate_quant": {
            "kernel": {"bf6": "rotquant_row_kernel<bf16,256,3 passes,B6T out> (one wave per row)",
                       "int8": "rotquant_row_kernel<bf16,256,3 passes,packed int4 out> (one wave per row)",
                       "w8a8": "rotquant_row_kernel<bf16,256,3 passes,I8T out> (one wave per row)"}[args.path],
            "bound": "hbm",
            # the metric point, burst-timed (see above); bytes as the metric counts
            # them (2 B read + 0.5 B written per element + 4 B per row)
            "us_at_M4608_K3072": round(rq_burst_us, 2),
            "GBps_at_M4608_K3072": round(rq_alg / rq_burst_us / 1e3, 1),
            "frac_at_M4608_K3072": round(rq_alg / rq_burst_us / 1e3 / PEAK_HBM_GBS, 4),
            # the same launch counting the bytes its output layout actually writes
            "GBps_at_M4608_K3072_layout_bytes": round(rq_alg_layout / rq_burst_us / 1e3, 1),
            # per-launch event intervals inside the step (each with its dispatch gap)
            "GBps_at_M4608_K3072_step_events": round(metric_rq_gbs, 1),
            "GBps_all_launches_step_events": round(rq_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "traffic": measured_traffic("rotquant_traffic_bytes_per_launch") if args.path == "bf6" else None,
        },
        "gemm_TOPS": round(gemm_tops, 1),
        "gemm_pct_int8_peak": round(100 * gemm_tops / PEAK_INT8_TOPS, 2),
        "detail": detail,
        "cpu_baseline": cpu,
        "cpu_baseline_c_oracle": cpu_c,
        "host_wall_s": round(wall, 3),
        "ms_per_step_with_kernel_events": round(ms_step_events, 4),
    }
    if copy_cal:
        line["copy_calibration"] = copy_cal
    print(json.dumps(line), flush=True)


RQ_SHAPES = ((4608, 3072), (4608, 12288), (16384, 3072), (16384, 12288))


def bench_rotquant(args):
    """The fused rotate + int4 quantize kernel alone, bf16 [M, K] in, at the
    block's M=4608 and the standalone M=16384 shapes: x ~ N(0,1) with 1% of
    channels replaced by Student-t(nu=3) draws at M=16384 (x20 outliers at
    M=4608), seed 0.  Both outputs: the packed int4 of the reference's C-ABI
    (ck_convrot_quant_int4) and the B6T operand of the product path.  Several
    input buffers in rotation (over 600 MB, beyond the 256 MB Infinity Cache);
    per launch, HIP events on the launch stream (queued behind about a
    millisecond of other GPU work so the launches run back to back), median
    over --steps.  GB/s =
    algorithmic bytes (2 B read + 0.5 B written per element + 4 B per row)
    over time."""
    import torch
    from inputs import outlier_activations
    importlib.import_module("comfyui-int4-convrot-rdna4_amd")
    native = importlib.import_module("comfyui-int4-convrot-rdna4_amd._int4.native")
    if not native.is_available():
        raise SystemExit("libconvrot_gfx950.so is not loadable on a gfx950 device; nothing to measure")
    lib = native.load_library()
    stream = torch.cuda.current_stream()
    sptr = ctypes.c_void_p(stream.cuda_stream)
    vp = ctypes.c_void_p
    lead = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    detail = {}
    for M, K in RQ_SHAPES:
        nbuf = max(2, (600 << 20) // (M * K * 2) + 1)
        base = outlier_activations(M, K, seed=0, student_t=(M == 16384))
        xs = [base.roll(i, 0).contiguous().cuda() for i in range(nbuf)]
        q = torch.empty((M, K // 2), dtype=torch.int8, device="cuda")
        a6 = torch.empty((native.bf6_rows(M), K // 4 * 3), dtype=torch.uint8, device="cuda")
        s = torch.empty((M,), dtype=torch.float32, device="cuda")
        for out, fn, dst in (("packed", lib.ck_convrot_quant_int4, q), ("b6t", lib.cr_convrot_quant_bf6, a6)):
            def launch(b):
                rc = fn(vp(xs[b % nbuf].data_ptr()), 1, vp(dst.data_ptr()), vp(s.data_ptr()), M, K, G, sptr)
                if rc != 0:
                    raise RuntimeError(f"rotate+quant launch failed rc={rc}")
            for b in range(args.warmup):
                launch(b)
            timer = HipTimer(args.steps + 1, stream.cuda_stream)
            torch.cuda.synchronize()
            gpu_lead(torch, lead)
            timer.record(0)
            for b in range(args.steps):
                launch(b)
                timer.record(b + 1)
            torch.cuda.synchronize()
            ts = sorted(timer.seconds(b, b + 1) for b in range(args.steps))
            timer.close()
            t = ts[len(ts) // 2]
            alg = rq_bytes(M, K, "int4")
            detail[f"{M}x{K} {out}"] = {"us": round(t * 1e6, 2), "GBps": round(alg / t / 1e9, 1),
                                         "frac": round(alg / t / 1e9 / PEAK_HBM_GBS, 4)}
        del xs
    head = detail["4608x3072 b6t"]
    line = {"metric": "rotate-quant GB/s (algorithmic bytes, packed-int4 count) at M=4608,K=3072",
            "value": head["GBps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(head["us"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "fused rotate + int4 quantize alone, bf16 [M, K], G=256",
                       "shapes": [list(x) for x in RQ_SHAPES]},
            "roofline": {"kernel": "rotquant_row_kernel (B6T out)", "bound": "hbm", "achieved": head["GBps"],
                         "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": head["frac"], "traffic": None},
            "detail": detail}
    print(json.dumps(line), flush=True)


SWEEP_M = (512, 1024, 2048, 4608, 8192, 16384)
SWEEP_KN = ((3072, 3072), (3072, 12288), (12288, 3072), (3840, 15360))


def bench_gemm_sweep(args):
    """The W4A4 GEMM alone (bf6 operands, bf16 output with bias) over the token
    sweep M x (K, N): int4 codes uniform in [-8, 7], scales U(0.005, 0.05),
    bias N(0, 0.01), seed 0; each shape timed over `--steps` launches with HIP
    events on the launch stream, k-split as the Linear replacement chooses it."""
    import numpy as np
    import torch
    importlib.import_module("comfyui-int4-convrot-rdna4_amd")
    native = importlib.import_module("comfyui-int4-convrot-rdna4_amd._int4.native")
    if not native.is_available():
        raise SystemExit("libconvrot_gfx950.so is not loadable on a gfx950 device; nothing to measure")
    lib = native.load_library()
    stream = torch.cuda.current_stream()
    sptr = ctypes.c_void_p(stream.cuda_stream)
    vp = ctypes.c_void_p
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    lead = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    detail, total_ops, total_s = {}, 0.0, 0.0
    for (K, N) in SWEEP_KN:
        w6 = native.int4_to_bf6(torch.randint(-128, 128, (N, K // 2), generator=g, device="cuda",
                                              dtype=torch.int8))
        ws = torch.rand(N, generator=g, device="cuda") * 0.045 + 0.005
        b = torch.randn(N, generator=g, device="cuda") * 0.01
        for M in SWEEP_M:
            a6 = native.int4_to_bf6(torch.randint(-128, 128, (M, K // 2), generator=g, device="cuda",
                                                  dtype=torch.int8))
            xs = torch.rand(M, generator=g, device="cuda") * 0.045 + 0.005
            out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
            ns = lib.cr_gemm_bf6_choose_nsplit(M, N, K)
            nb = lib.cr_gemm_bf6_splitk_workspace(M, N, ns)
            wsp = torch.zeros((max(nb, 2048),), dtype=torch.uint8, device="cuda")   # split counters start at 0
            call = (vp(a6.data_ptr()), vp(w6.data_ptr()), vp(xs.data_ptr()), vp(ws.data_ptr()), vp(b.data_ptr()),
                    None, None, 0, ctypes.c_float(0.0), vp(out.data_ptr()), M, N, K, 1, ns, vp(wsp.data_ptr()),
                    nb, sptr)
            for _ in range(args.warmup):
                assert lib.cr_int4_convrot_gemm_bf6_splitk(*call) == 0
            timer = HipTimer(args.steps + 1, stream.cuda_stream)
            torch.cuda.synchronize()
            gpu_lead(torch, lead)
            timer.record(0)
            for r in range(args.steps):
                assert lib.cr_int4_convrot_gemm_bf6_splitk(*call) == 0
                timer.record(r + 1)
            torch.cuda.synchronize()
            us = sorted(timer.seconds(r, r + 1) * 1e6 for r in range(args.steps))
            timer.close()
            med = us[len(us) // 2]
            ops = 2.0 * M * N * K
            bm, bn = native.gemm_tile_bf6(M, N, K, ns)
            detail[f"{M}x{K}->{N}"] = {"us": round(med, 2), "TOPS": round(ops / med / 1e6, 1), "nsplit": ns,
                                       "tile": f"{bm}x{bn}"}
            total_ops += ops
            total_s += med * 1e-6
            del a6, out, wsp
    line = {
        "metric": "W4A4 GEMM token sweep: effective int4 TOPS (%int8 MFMA peak)",
        "value": round(total_ops / total_s / 1e12, 1),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_s * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # the path's arithmetic: int4 codes (int8 codes for the W8A8 tier) with exact
        # integer accumulation; the products run on BF6 / int8 matrix cores
        "dtype": "int8" if args.path == "w8a8" else "int4",
        "data": "synthetic",
        "config": {"workload": "W4A4 GEMM token sweep, bf6 operands, bf16 out + bias: M in %s x (K, N) in %s; codes "
                               "uniform [-8, 7], scales U(0.005, 0.05)" % (list(SWEEP_M), [list(x) for x in SWEEP_KN])},
        "pct_int8_peak": round(100 * total_ops / total_s / 1e12 / PEAK_INT8_TOPS, 2),
        "detail": detail,
    }
    print(json.dumps(line), flush=True)


DIT_IMG, DIT_TXT, DIT_DEPTH, DIT_RANK = 4096, 512, 8, 32


def bench_dit(args):
    """The synthetic 8-block double-stream DiT stack (hidden 3072, 24 heads,
    MLP ratio 4; 4096 image + 512 text tokens) loaded through Int4ConvRotOps
    with the Flux 2 skip list and a rank-32 dynamic LoRA on each of its 64
    quantized linears.  One step = one forward.  Reports the forward time, the
    same forward captured in a HIP graph and replayed (bits checked against the
    eager forward), the GPU time inside the quantized linears (HIP events
    around each call), the
    same linears replayed back to back through the C-ABI's one-call linear
    (with and without the LoRA: their difference is the LoRA's cost) and the
    difference between the two: the per-layer cost of the Linear replacement's
    host path (casts, allocation, launch gaps)."""
    import torch
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import dit_stack as ds
    from fake_comfy import FakeLoRA, install_fake_comfy
    install_fake_comfy()
    importlib.import_module("comfyui-int4-convrot-rdna4_amd")
    native = importlib.import_module("comfyui-int4-convrot-rdna4_amd._int4.native")
    if not native.is_available():
        raise SystemExit("libconvrot_gfx950.so is not loadable on a gfx950 device; nothing to measure")
    ops_mod = importlib.import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if ops_mod.Int4ConvRotOps is None:
        ops_mod = importlib.reload(ops_mod)
    Ops = ops_mod.Int4ConvRotOps

    t0 = time.perf_counter()
    model, _, patches, applied = ds.build_int4_stack(Ops, FakeLoRA, depth=DIT_DEPTH, n_lora_rank=DIT_RANK,
                                                     keep_reference=False)
    torch.cuda.synchronize()
    load_s = time.perf_counter() - t0
    qlayers = [(n, m) for n, m in model.named_modules() if hasattr(m, "in_features") and ds.is_quantized_name(n)]
    assert all(m._qmode == "int4" and m._dyn_fused is not None for _, m in qlayers) and applied == set(patches)
    img, ctx, tt = ds.synthetic_inputs(DIT_IMG, DIT_TXT, device="cuda")
    stream = torch.cuda.current_stream()

    with torch.no_grad():
        for _ in range(args.warmup):
            model(img, ctx, tt)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        h0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            model(img, ctx, tt)
        e1.record(stream)
        host_s = (time.perf_counter() - h0) / args.steps
        torch.cuda.synchronize()
        ms_fwd = e0.elapsed_time(e1) / args.steps

        # the same forward captured once in a HIP graph and replayed: no host
        # work per launch (the Linear replacement's Python path included); the
        # replay's output is checked against the eager forward's bits
        static = [img.clone(), ctx.clone(), tt.clone()]
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            model(*static)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            gout = model(*static)
        graph.replay()
        eager_out = model(img, ctx, tt)
        torch.cuda.synchronize()
        graph_exact = bool(torch.equal(gout.view(torch.int16), eager_out.view(torch.int16)))
        e0.record(stream)
        for _ in range(args.steps):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        ms_graph = e0.elapsed_time(e1) / args.steps
        del graph, gout, eager_out, static

        # GPU time inside the quantized linears: events around each call
        evs, inputs = [], {}

        def pre(mod, a, name):
            ev = torch.cuda.Event(enable_timing=True)
            ev.record(torch.cuda.current_stream())
            evs.append([name, ev, None])
            inputs.setdefault(name, a[0])

        def post(mod, a, out):
            ev = torch.cuda.Event(enable_timing=True)
            ev.record(torch.cuda.current_stream())
            evs[-1][2] = ev

        hooks = []
        for n, m in qlayers:
            hooks.append(m.register_forward_pre_hook(lambda mod, a, n=n: pre(mod, a, n)))
            hooks.append(m.register_forward_hook(post))
        n_instr = 3
        for _ in range(n_instr):
            model(img, ctx, tt)
        torch.cuda.synchronize()
        for h in hooks:
            h.remove()
        lin_ms = sum(a.elapsed_time(b) for _, a, b in evs) / n_instr

        # the same linears replayed back to back through the C-ABI's one-call
        # linear (the Linear's own launches: LoRA partial sums, rotate+quant
        # with the LoRA sum, GEMM with the LoRA epilogue), with and without the
        # LoRA; one HIP event after every call
        lib = native.load_library()
        sptr = ctypes.c_void_p(stream.cuda_stream)
        vp = ctypes.c_void_p
        calls = []
        keep = []
        for n, m in qlayers:
            x = inputs[n].reshape(-1, m.in_features).contiguous()
            M, K, N = x.shape[0], m.in_features, m.out_features
            D, U = m._dyn_fused
            R = D.shape[0]
            out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
            b32 = m.bias.float().contiguous()
            nb = lib.cr_convrot_w4a4_linear_bf6_workspace(M, N, K, R)
            wsp = torch.zeros((max(nb, 2048),), dtype=torch.uint8, device="cuda")   # split counters start at 0
            keep += [x, out, b32, wsp]
            for kind, r in (("linear_lora", R), ("linear_plain", 0)):
                calls.append((kind, lib.cr_convrot_w4a4_linear_bf6,
                              (vp(x.data_ptr()), 1, vp(m._q6.data_ptr()), vp(m._qs.data_ptr()), vp(b32.data_ptr()),
                               0, vp(D.data_ptr()) if r else None, vp(U.data_ptr()) if r else None, r,
                               ctypes.c_float(1.0), vp(out.data_ptr()), 1, M, N, K, m._qgs, vp(wsp.data_ptr()), nb,
                               sptr)))
        # all the LoRA calls over the 64 layers, then all the plain ones: each
        # call then finds the previous layer's data in the caches, not its own
        calls.sort(key=lambda c: c[0] != "linear_lora")
        kern = {}
        reps = 3
        timer = HipTimer(len(calls) + 1, stream.cuda_stream)
        for rep in range(reps + 1):
            torch.cuda.synchronize()
            timer.record(0)
            for c, (kind, fn, a) in enumerate(calls):
                rc = fn(*a)
                timer.record(c + 1)
                if rc != 0:
                    raise RuntimeError(f"{kind} launch failed rc={rc}")
            torch.cuda.synchronize()
            if rep > 0:
                for c, (kind, _, _) in enumerate(calls):
                    kern[kind] = kern.get(kind, 0.0) + timer.seconds(c, c + 1) * 1e3 / reps
        timer.close()
        del keep

    work = ds.quantized_work(DIT_IMG, DIT_TXT, depth=DIT_DEPTH)
    work_lora = ds.quantized_work(DIT_IMG, DIT_TXT, depth=DIT_DEPTH, lora_rank=DIT_RANK)
    kern_ms = kern["linear_lora"]
    line = {
        "metric": "DiT stack forward: quantized-linear TOPS inside the forward (8 double blocks, LoRA r32)",
        "value": round(work / (lin_ms * 1e-3) / 1e12, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_fwd, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # the path's arithmetic: int4 codes (int8 codes for the W8A8 tier) with exact
        # integer accumulation; the products run on BF6 / int8 matrix cores
        "dtype": "int8" if args.path == "w8a8" else "int4",
        "data": "synthetic",
        "config": {
            "workload": "synthetic double-stream DiT stack through Int4ConvRotOps: 8 blocks, hidden 3072, 24 heads, "
                        "MLP ratio 4, 4096 image + 512 text tokens, Flux 2 skip list kept bf16, rank-32 dynamic "
                        "LoRA fused on the 64 quantized linears, weights N(0, 0.02)",
            "image_tokens": DIT_IMG, "text_tokens": DIT_TXT, "depth": DIT_DEPTH, "lora_rank": DIT_RANK,
            "quantized_linears": len(qlayers),
        },
        "forward_ms": round(ms_fwd, 3),
        "forward_graph_ms": round(ms_graph, 3),
        "graph_replay_bit_exact": graph_exact,
        "host_ms_per_forward": round(host_s * 1e3, 3),
        "quantized_linear_ms": round(lin_ms, 3),
        "other_ms": round(ms_fwd - lin_ms, 3),
        "kernels_ms": {k: round(v, 3) for k, v in kern.items()},
        "kernel_only_linear_ms": round(kern_ms, 3),
        "linear_overhead_ms": round(lin_ms - kern_ms, 3),
        "linear_overhead_us_per_layer": round((lin_ms - kern_ms) * 1e3 / len(qlayers), 2),
        "lora_cost_ms": round(kern["linear_lora"] - kern["linear_plain"], 3),
        "quantized_TOP_per_forward": round(work / 1e12, 3),
        "quantized_TOP_per_forward_with_lora": round(work_lora / 1e12, 3),
        "kernel_only_TOPS": round(work / (kern_ms * 1e-3) / 1e12, 1),
        "load_s": round(load_s, 2),
    }
    print(json.dumps(line), flush=True)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_torch(target_s: float):
    """The reference's eager CPU path, restated with the same torch operations
    (oracle/torch_eager.py; it reproduces the reference eager output bit for
    bit): for each of the block's four linears, bf16 rotation matmul, bf16
    rowwise quantize + nibble pack, unpack + bf16 int-code matmul + bf16
    epilogue, on the first rows of the token batch (weights quantized from fp16
    beforehand, untimed).  torch's intra-op threads (the box's CPU share); one
    warm-up, then the median of three repetitions, with per-stage times and
    rates in the GPU's units (rotate+quant GB/s, GEMM TOPS)."""
    import torch
    from oracle import torch_eager as te
    from inputs import normal_bias, normal_weight, outlier_activations

    layers = []
    for i, (name, K, N) in enumerate(LINEARS):
        qw, ws = te.quantize_weight(normal_weight(N, K, seed=11 + i), G)
        layers.append((K, N, qw, ws, normal_bias(N, seed=21 + i)))
    threads = torch.get_num_threads()

    x_all = [outlier_activations(M_TOKENS, K, seed=K) for K, *_ in layers]

    def run(rows):
        stages = {}
        t0 = time.perf_counter()
        for x, (K, N, qw, ws, bias) in zip(x_all, layers):
            te.linear(x[:rows], qw, ws, bias, G, stage_seconds=stages)
        return time.perf_counter() - t0, stages

    probe = 256
    run(16)                                             # first-call set-up
    t, _ = run(probe)                                   # size probe
    rows = int(max(probe, min(M_TOKENS, probe * (target_s / 4) / max(t, 1e-6))))
    rows -= rows % 16
    run(rows)                                           # warm-up at the sample size
    reps = sorted((run(rows) for _ in range(3)), key=lambda r: r[0])
    t, stages = reps[1]
    ops = 2.0 * rows * sum(N * K for _, K, N in LINEARS)
    rq_b = sum(rq_bytes(rows, K, "int4") for _, K, _ in LINEARS)
    t_rq = stages["rotate"] + stages["quantize_pack"]
    cpu = _cpu_model()
    return {"value": round(ops / t / 1e12, 6), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"torch restatement of the reference eager path (bf16 rotation matmul, bf16 quantize + "
                      f"pack, bf16 int-code matmul + epilogue; {threads} torch threads on {cpu}): {rows} of the "
                      f"{M_TOKENS} rows through the block's four linears; median of 3 repetitions after "
                      f"warm-up",
            "seconds": round(t, 3),
            "stage_seconds": {k: round(v, 3) for k, v in stages.items()},
            "rotate_quant_GBps": round(rq_b / t_rq / 1e9, 2),
            "gemm_TOPS": round(ops / stages["gemm_epilogue"] / 1e12, 4),
            "cpu_model": cpu}


def cpu_baseline(target_s: float):
    """The oracle (plain C, row loops in parallel with OpenMP over the host
    cores it is given) on a bounded sample of the same step: the first rows of
    the token batch through all four linears of the block (rotate+quant, exact
    integer GEMM, fp32 epilogue to bf16).  One warm-up, then the median of
    three timed repetitions, with per-stage times; reported in the same unit
    (effective TOPS)."""
    import numpy as np
    import torch
    import oracle
    from inputs import bf16_bits, normal_weight, outlier_activations

    layers = []
    for i, (name, K, N) in enumerate(LINEARS):
        w = normal_weight(N, K, seed=11 + i).view(torch.int16).numpy().view(np.uint16)
        qw, ws = oracle.quantize_weight(w, oracle.F16, G)
        layers.append((K, N, qw, ws, np.zeros(N, dtype=np.float32)))
    threads = oracle.num_threads()

    def run(rows):
        xs_in = [bf16_bits(outlier_activations(rows, K, seed=rows + K)) for K, *_ in layers]
        st = [0.0, 0.0, 0.0]
        for x, (K, N, qw, ws, bias) in zip(xs_in, layers):
            t0 = time.perf_counter()
            q, xs, _ = oracle.rotquant(x, oracle.BF16, G)
            t1 = time.perf_counter()
            acc = oracle.int_gemm(q, qw)
            t2 = time.perf_counter()
            oracle.epilogue_f32(acc, xs, ws, bias, out_bf16=True)
            t3 = time.perf_counter()
            st[0] += t1 - t0
            st[1] += t2 - t1
            st[2] += t3 - t2
        return sum(st), st

    probe = 8 * max(1, threads)
    t, _ = run(probe)                                   # warm-up and size probe
    rows = int(max(probe, min(M_TOKENS, probe * (target_s / 3) / max(t, 1e-6))))
    reps = sorted((run(rows) for _ in range(3)), key=lambda r: r[0])
    t, (t_rq, t_gemm, t_epi) = reps[1]
    ops = 2.0 * rows * sum(N * K for _, K, N in LINEARS)
    cpu = _cpu_model()
    return {"value": round(ops / t / 1e12, 6), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"oracle (C, OpenMP, {threads} threads on {cpu}): {rows} of the {M_TOKENS} rows "
                      f"through the block's four linears (rotate+quant, int GEMM, epilogue); "
                      f"median of 3 repetitions after one warm-up",
            "seconds": round(t, 3),
            "stage_seconds": {"rotate_quant": round(t_rq, 3), "gemm": round(t_gemm, 3),
                              "epilogue": round(t_epi, 3)},
            "cpu_model": cpu}


if __name__ == "__main__":
    main()
