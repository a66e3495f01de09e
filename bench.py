"""Benchmark of the fused INT8 convrot linear on one MI355X.

Workload (one step = one pass of the hot path over one batch): the DiT fused QKV projection, M=32768 tokens,
K=5120, N=15360, Hadamard group 256, low-rank rank 64, no bias, synthetic seeded data resident in HBM:
x bf16 N(0,1) with 0.5% outlier channels x30, qweight int8 U{-127..127}, wscale fp32 U(1e-3, 1e-2), low-rank
down/up bf16 N(0, 0.02). A step is the whole fused layer: rotate+quantize, low-rank down projection, INT8 GEMM with
the fused epilogue.

value = 2*M*N*K int8 ops per step / measured step time (TOPS). The roofline object is for the dominant kernel
(the GEMM): its average duration comes from HIP events recorded around every GEMM launch on the launch stream inside
the timed region. The CPU baseline times the PyTorch-CPU path of the reference layer on a bounded row sample of the
same workload on this host.

`--config N` runs one of the other measured workloads instead and prints one JSON line per shape (these are
parity-test shapes and supporting measurements, not the headline line):
  1  M=1024 K=3072 N=3072, rank 32, bias, 1% outlier channels x20
  3  FFN pair on M=32768: up 5120->13824, tanh-GELU in bf16, down 13824->5120, rank 64
  4  one DiT block's linears on M=41344: QKV 5120->15360, out 5120->5120, up 5120->13824, down 13824->5120, rank 64
  5  small M in {64, 256, 1024}, K=5120, N in {5120, 30720}, rank 32: HBM GB/s over the compulsory bytes, with
     enough weight copies rotated per step that the weights come from HBM, not the 256 MiB Infinity Cache; the
     layer calls are captured in a HIP graph and replayed (the per-call host work would otherwise dominate)
  6  the model's gated FFN on M=32768: up 5376->28672 (14336 hidden + 14336 gate rows), SwiGLU in bf16, down
     14336->5376, rank 64; timed unfused (torch chunk + silu + multiply between the layers) and fused (SwiGLU in
     the up-projection's GEMM epilogue)
  7  the model's own linear shapes (K, N) on the 5.2 s clip's M=37710 tokens, rank 64: q/k/v 5376->7168 each,
     the fused q/k/v 5376->21504, out 7168->5376, gated up 5376->28672, down 14336->5376
  8  the standalone low-rank linear up(down(x)) (the model's non-INT8 linears) at M=37710, K->N 5376->7168 and
     14336->5376, ranks 64, 256 and 512: TFLOP/s of 2 M r (K + N), with the vendor library's bf16 GEMMs beside it
     (the two alternate over three rounds; each reports its median round)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--config N [--rows M]]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

M, K, N, GROUP, RANK = 32768, 5120, 15360, 256, 64
PEAK_INT8_TOPS = 5033.2  # MI355X dense INT8 MFMA: 256 CUs x 2.4 GHz x 8192 ops/clk
PEAK_HBM_GBS = 8000.0
METRIC = "convrot INT8 linear TOPS + % of MI355X INT8 MFMA peak, M=32768 K=5120"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_int8_gemm_qkv_m32768.txt")


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-rows", type=int, default=32768, help="row sample for the CPU baseline")
    p.add_argument("--config", type=int, default=2, choices=(1, 2, 3, 4, 5, 6, 7, 8),
                   help="workload: 2 (default) is the headline QKV projection; 1, 3-8 are supporting measurements")
    p.add_argument("--rows", type=int, default=None,
                   help="--config 5: only this M (64, 256 or 1024); --config 4: this many tokens (default 41344)")
    p.add_argument("--copy-probe", action="store_true",
                   help="only copy a 1 GiB device buffer 3 times (calibrates the HBM byte counters) and exit")
    p.add_argument("--ceilings", action="store_true",
                   help="only measure the device's ceilings (INT8 MFMA with no memory traffic, a device copy's "
                        "bandwidth) and exit; the headline run reports them too")
    p.add_argument("--operand-sweep", action="store_true",
                   help="time the headline GEMM (same kernel, rank-64 epilogue) on operand sets of different bit "
                        "toggling: the bench's codes and weights, all zero, all one, narrow codes, zero weights")
    p.add_argument("--vendor-gemm", action="store_true",
                   help="only time the vendor library's own INT8, FP8 and bf16 GEMMs at the headline shape (a "
                        "calibration of what the matrix cores sustain, not this build's path) and exit")
    return p.parse_args()


def vendor_gemm(torch, steps, warmup):
    """hipBLASLt (through torch) at M=32768 N=15360 K=5120: INT8 -> INT32, FP8 e4m3fn -> bf16, bf16 -> bf16."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    m, n, k = M, N, K
    cases = {}
    a8 = torch.randint(-127, 128, (m, k), device=dev, generator=gen, dtype=torch.int8)
    b8 = torch.randint(-127, 128, (n, k), device=dev, generator=gen, dtype=torch.int8)
    cases["int8_int_mm"] = lambda: torch._int_mm(a8, b8.t())
    af = torch.randn(m, k, device=dev, generator=gen).to(torch.float8_e4m3fn)
    bf = torch.randn(n, k, device=dev, generator=gen).to(torch.float8_e4m3fn)
    one = torch.ones((), device=dev)
    cases["fp8_e4m3fn_scaled_mm"] = lambda: torch._scaled_mm(af, bf.t(), scale_a=one, scale_b=one,
                                                             out_dtype=torch.bfloat16)
    ab = torch.randn(m, k, device=dev, generator=gen, dtype=torch.bfloat16)
    bb = torch.randn(n, k, device=dev, generator=gen, dtype=torch.bfloat16)
    cases["bf16_matmul"] = lambda: ab @ bb.t()
    for name, fn in cases.items():
        t = timed(torch, fn, steps, warmup)
        print(json.dumps({"vendor_gemm": name, "M": m, "N": n, "K": k, "us": round(t * 1e6, 1),
                          "tera_ops": round(2.0 * m * n * k / t / 1e12, 1)}), flush=True)


def copy_probe(torch):
    """Three device-to-device copies of 1 GiB: the known-size workload that scales FETCH_SIZE / WRITE_SIZE."""
    dev = torch.device("cuda:0")
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_per_launch": src.numel() * 4}), flush=True)


def ceilings(torch, repeats=5):
    """Measured ceilings of this device, beside the published peaks: the INT8 matrix cores' rate with no memory
    traffic (libhf_ceilings.so, one 8-wave workgroup per CU issuing independent v_mfma_i32_32x32x32_i8) on zero
    operands and on uniform random codes, whose bit toggling sets the clock the chip holds, the bandwidth of a
    1 GiB device-to-device copy (read + write bytes), and of streaming passes over 1 GiB (libhf_ceilings.so
    stream_kernel) at the rotation's 2:1 read:write ratio and read-only, the best of a sweep of launch shapes. Each
    figure is the mean of `repeats` launches after two."""
    from hyperflow_h3_flash_amd import _native

    lib = _native.ceilings_library()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    rounds, grid = 12000, cus
    out = torch.empty(grid * 512, dtype=torch.int32, device=dev)

    def mean_seconds(launch):
        for _ in range(2):
            launch()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        e[0].record(stream)
        for _ in range(repeats):
            launch()
        e[1].record(stream)
        torch.cuda.synchronize()
        return e[0].elapsed_time(e[1]) * 1e-3 / repeats

    result = {}
    tables = {"zero": torch.zeros(8192, dtype=torch.int8, device=dev),
              "uniform": torch.randint(-127, 128, (8192,), dtype=torch.int8, device=dev, generator=gen)}
    ops = 2.0 * lib.hf_ceiling_mfma_i8_macs(rounds, grid)
    for name, table in tables.items():
        def launch():
            rc = lib.hf_ceiling_mfma_i8(table.data_ptr(), rounds, grid, out.data_ptr(), stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"hf_ceiling_mfma_i8 failed: {rc}")
        t = mean_seconds(launch)
        result[f"mfma_int8_{name}_TOPS"] = round(ops / t / 1e12, 1)
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    t = mean_seconds(lambda: dst.copy_(src))
    result["copy_GBs"] = round(2.0 * src.numel() * 4 / t / 1e9, 1)
    # Streaming passes over 1 GiB of source (libhf_ceilings.so stream_kernel), the best of a sweep of grid sizes
    # and unrolls: 2 bytes read per byte written (the rotation's ratio), read-only (the low-rank projection's).
    units = (1 << 30) // 32
    sink = torch.empty(cus * 16 * 256, dtype=torch.int32, device=dev)
    for name, (reads, writes) in {"stream_r2w1_GBs": (2, 1), "stream_read_GBs": (2, 0)}.items():
        best = 0.0
        for grid in (cus * 2, cus * 4, cus * 8, cus * 16):
            for unroll in (4, 8):
                def launch():
                    rc = lib.hf_ceiling_stream(src.data_ptr(), dst.data_ptr() if writes else None, units, reads,
                                               writes, unroll, grid, sink.data_ptr(), stream.cuda_stream)
                    if rc != 0:
                        raise RuntimeError(f"hf_ceiling_stream failed: {rc}")
                t = mean_seconds(launch)
                best = max(best, units * 16 * (reads + writes) / t / 1e9)
        result[name] = round(best, 1)
    del src, dst, sink
    return result


def gemm_operand_sets(torch, dev, xq, qweight):
    """Operand sets for the headline GEMM that differ only in how many operand bits toggle: the bench's own codes
    (rotated activations) and weights, all zero, all one (constant bits), codes and weights uniform in [-20, 20],
    and the bench's codes against zero weights. The GEMM's dataflow (loads, LDS traffic, MFMA count, epilogue and
    stores) is the same for every set."""
    gen = torch.Generator(device=dev).manual_seed(11)
    return {
        "bench": (xq, qweight),
        "zero": (torch.zeros_like(xq), torch.zeros_like(qweight)),
        "ones": (torch.ones_like(xq), torch.ones_like(qweight)),
        "narrow": (torch.randint(-20, 21, xq.shape, device=dev, dtype=torch.int8, generator=gen),
                   torch.randint(-20, 21, qweight.shape, device=dev, dtype=torch.int8, generator=gen)),
        "zero_weights": (xq, torch.zeros_like(qweight)),
    }


def operand_sweep(torch, rounds=5, calls=4):
    """The headline GEMM (M=32768, K=5120, N=15360, rank-64 epilogue) on each of gemm_operand_sets, interleaved
    round by round after a warm-up, HIP events on the launch stream; one JSON line of median microseconds per call
    and TOPS. Under `rocprofv3 --pmc` the launches come in a fixed order: 2 warm-up calls per set, then per round
    `calls` calls of each set in the order of the dict."""
    from hyperflow_h3_flash_amd.int8 import _kernels

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    kernels = _kernels()
    x, qweight, wscale, down, up = make_inputs(torch, dev)
    with torch.no_grad():
        xq, sx = kernels.rotate_quant(x, GROUP)
        u = kernels.lowrank_down(x, down)
    del x
    sets = gemm_operand_sets(torch, dev, xq, qweight)
    stream = torch.cuda.current_stream(dev)
    times = {name: [] for name in sets}
    for q, w in sets.values():
        for _ in range(2):
            kernels.int8_matmul(q, w, sx, wscale, u=u, up=up)
    torch.cuda.synchronize()
    for _ in range(rounds):
        for name, (q, w) in sets.items():
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(calls):
                kernels.int8_matmul(q, w, sx, wscale, u=u, up=up)
            e1.record(stream)
            torch.cuda.synchronize()
            times[name].append(e0.elapsed_time(e1) * 1e3 / calls)
    ops = 2.0 * M * N * K
    us = {name: round(statistics.median(v), 1) for name, v in times.items()}
    print(json.dumps({"operand_sweep_us": us,
                      "operand_sweep_TOPS": {name: round(ops / (t * 1e-6) / 1e12, 1) for name, t in us.items()},
                      "config": {"M": M, "K": K, "N": N, "rank": RANK}}), flush=True)


def make_inputs(torch, dev, seed=0):
    gen = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, device=dev, generator=gen)
    cols = torch.randperm(K, device=dev, generator=gen)[: -(-K * 5 // 1000)]
    x[:, cols] *= 30.0
    x = x.to(torch.bfloat16)
    qweight = torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8, generator=gen)
    wscale = torch.rand(N, device=dev, generator=gen) * 9e-3 + 1e-3
    down = (torch.randn(RANK, K, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
    up = (torch.randn(N, RANK, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
    return x, qweight, wscale, down, up


def read_traffic():
    """HBM bytes per GEMM launch from the committed rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, scaled by the
    copy-kernel calibration), or None when no summary is committed."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def onednn_isa() -> str:
    """The instruction set oneDNN dispatches bf16 matmuls to on this host, from its verbose log of one small bf16
    matmul run in a child process (ONEDNN_VERBOSE=1); "unknown" when the log has no ISA line."""
    import subprocess

    code = "import torch; a = torch.randn(64, 64).to(torch.bfloat16); (a @ a).sum()"
    try:
        out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120,
                             env=dict(os.environ, ONEDNN_VERBOSE="1", DNNL_VERBOSE="1")).stdout
    except (OSError, subprocess.SubprocessError):
        return "unknown"
    for line in out.splitlines():
        if ",info,cpu,isa:" in line:
            return line.split("isa:", 1)[1].strip()
    return "unknown"


_HOST = {}


def host_description(torch) -> str:
    if not _HOST:
        _HOST["text"] = (f"torch {torch.__version__} CPU on {cpu_model()}; ATen CPU capability "
                         f"{torch.backends.cpu.get_cpu_capability()}; oneDNN ISA {onednn_isa()}")
    return _HOST["text"]


def cpu_baseline(torch, rows, seed=0, m=M, k=K, n=N, rank=RANK, bias=False, outlier_frac=0.005,
                 outlier_scale=30.0, chain=None):
    """The reference's CPU PyTorch path (int8.py:173-179, restated in oracle/torch_path.py) plus the low-rank
    composition (and a bias), on a `rows`-row sample of an m-row workload with the same input distributions (x
    N(0,1) with ceil(outlier_frac * K) outlier channels scaled by outlier_scale): 1 warm-up then the median of 3
    timed calls. `chain` lists further (K, N, source) layers: source "gelu_tanh" applies torch's tanh-GELU to the
    previous layer's output and feeds it (an FFN pair), "x" gives the layer its own seeded input of width K (the
    other linears of a block); the ops of every layer are counted."""
    from oracle import torch_path

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(seed)

    def weights(kk, nn):
        qweight = torch.randint(-127, 128, (nn, kk), dtype=torch.int8, generator=gen)
        wscale = torch.rand(nn, generator=gen) * 9e-3 + 1e-3
        down = (torch.randn(rank, kk, generator=gen) * 0.02).to(torch.bfloat16) if rank else None
        up = (torch.randn(nn, rank, generator=gen) * 0.02).to(torch.bfloat16) if rank else None
        b = (torch.randn(nn, generator=gen) * 0.01).to(torch.bfloat16) if bias else None
        return qweight, wscale, down, up, b

    def activations(kk):
        x = torch.randn(rows, kk, generator=gen)
        cols = torch.randperm(kk, generator=gen)[: -(-int(round(outlier_frac * 1e4)) * kk // 10000)]
        x[:, cols] *= outlier_scale
        return x.to(torch.bfloat16)

    inputs = {}
    layers = [(k, n, "x", weights(k, n))] + [(kk, nn, src, weights(kk, nn)) for kk, nn, src in (chain or [])]
    for kk, _, src, _ in layers:
        if src == "x" and kk not in inputs:
            inputs[kk] = activations(kk)

    def run():
        h = None
        for kk, nn, src, (qw, ws, dn, upw, b) in layers:
            src_x = torch.nn.functional.gelu(h, approximate="tanh") if src == "gelu_tanh" else inputs[kk]
            h = torch_path.forward_torch(src_x, qw, ws, GROUP, dn, upw, b)
        return h

    times = []
    for i in range(4):
        t0 = time.perf_counter()
        run()
        t = time.perf_counter() - t0
        if i:
            times.append(t)
    t = statistics.median(times)
    ops = sum(2.0 * rows * nn * kk for kk, nn, _, _ in layers)
    shapes = ", ".join(f"K={kk} N={nn}" for kk, nn, _, _ in layers)
    return {
        "value": round(ops / t / 1e12, 4),
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"{rows} of {m} rows ({shapes}, G={GROUP}, rank {rank}{', bias' if bias else ''}, "
                  f"{outlier_frac * 100:g}% outlier channels x{outlier_scale:g}); median of 3 after 1 warm-up, "
                  f"{t:.3f} s per call; {host_description(torch)}",
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (one MI355X per run; the linear "
              "shards by rows with no communication, so N GPUs run N independent copies)", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.vendor_gemm:
        vendor_gemm(torch, args.steps, args.warmup)
        return
    if args.copy_probe:
        copy_probe(torch)
        return
    if args.operand_sweep:
        operand_sweep(torch)
        return
    if args.ceilings:
        print(json.dumps({"ceilings": ceilings(torch), "published": {"mfma_int8_TOPS": PEAK_INT8_TOPS,
                                                                      "hbm_GBs": PEAK_HBM_GBS}}), flush=True)
        return
    if args.config != 2:
        for line in run_config(torch, args.config, args.steps, args.warmup, rows=args.rows,
                               cpu_rows=0 if args.no_cpu_baseline else args.cpu_rows):
            print(json.dumps(line), flush=True)
        return

    from hyperflow_h3_flash_amd import Int8RotLinear
    from hyperflow_h3_flash_amd.int8 import _kernels

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    x, qweight, wscale, down, up = make_inputs(torch, dev)
    layer = Int8RotLinear(K, N, GROUP, rank=RANK).to(dev)
    with torch.no_grad():
        layer.qweight.copy_(qweight)
        layer.wscale.copy_(wscale)
        layer.down.weight.copy_(down)
        layer.up.weight.copy_(up)
    del qweight, wscale
    kernels = _kernels()
    stream = torch.cuda.current_stream(dev)

    # per-kernel events on the launch stream (torch's current stream). Each event record costs the stream ~4-5 us, so
    # the timed steps record only the GEMM's pair (the roofline's kernel); the rotation's and the low-rank pass's own
    # durations come from a few steps with events around every kernel after the timed region.
    ev = {name: [] for name in ("rotate", "lowrank", "gemm")}

    def step(record):
        """One step; record: None, "gemm" (events around the GEMM) or "all" (around each of the three kernels)."""
        with torch.no_grad():
            e = [torch.cuda.Event(enable_timing=True) for _ in range(4)] if record else None
            if record == "all":
                e[0].record(stream)
            xq, sx = kernels.rotate_quant(x, GROUP)
            if record == "all":
                e[1].record(stream)
            u = kernels.lowrank_down(x, layer.down.weight)
            if record:
                e[2].record(stream)
            y = kernels.int8_matmul(xq, layer.qweight, sx, layer.wscale, u=u, up=layer.up.weight)
            if record:
                e[3].record(stream)
                if record == "all":
                    ev["rotate"].append((e[0], e[1]))
                    ev["lowrank"].append((e[1], e[2]))
                else:
                    ev["gemm"].append((e[2], e[3]))
        return y

    # the timed step is exactly what Int8RotLinear.forward launches for a bf16 [M, K] input
    with torch.no_grad():
        torch.testing.assert_close(step(False), layer(x), rtol=0, atol=0)
    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step("gemm")
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    for _ in range(min(args.steps, 10)):
        step("all")
    torch.cuda.synchronize()

    ops = 2.0 * M * N * K
    ms_per_step = elapsed / args.steps * 1e3
    tops = ops * args.steps / elapsed / 1e12
    avg_us = {k: statistics.mean(a.elapsed_time(b) for a, b in v) * 1e3 for k, v in ev.items()}
    gemm_tops = ops / (avg_us["gemm"] * 1e-6) / 1e12
    rotate_bytes = 2 * M * K + M * K + 4 * M
    result = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded: x N(0,1) with 0.5% outlier channels x30, uniform int8 weights; resident in HBM)",
        "config": {"workload": "DiT fused QKV convrot linear: rotate+quant, low-rank down, INT8 GEMM + fused "
                               "epilogue", "M": M, "K": K, "N": N, "group": GROUP, "rank": RANK, "bias": False},
        "pct_of_peak": round(100.0 * tops / PEAK_INT8_TOPS, 2),
        "kernel_us": {k: round(v, 2) for k, v in avg_us.items()},
        "kernel_us_from": "gemm: events around it in every timed step; rotate, lowrank: events around every kernel "
                          "in up to 10 steps after the timed region",
        "rotate_quant_GBs": round(rotate_bytes / (avg_us["rotate"] * 1e-6) / 1e9, 1),
        "lowrank_down_GBs": round((2 * M * K + 2 * M * RANK) / (avg_us["lowrank"] * 1e-6) / 1e9, 1),
        "roofline": {
            "bound": "mfma",
            "achieved": round(gemm_tops, 2),
            "peak": PEAK_INT8_TOPS,
            "unit": "TOPS",
            "frac": round(gemm_tops / PEAK_INT8_TOPS, 4),
            "traffic": read_traffic(),
        },
        "cpu_baseline": None,
    }
    # The GEMM's rate against what the matrix cores hold on random codes with no memory traffic, and the rotation
    # pass against a device copy's bandwidth (measured after the timed region).
    ceil = ceilings(torch)
    ceil["gemm_frac_of_mfma_uniform"] = round(gemm_tops / ceil["mfma_int8_uniform_TOPS"], 4)
    # The same GEMM call (same kernel, dataflow and epilogue) with all-zero codes and weights: the rate of this
    # dataflow when the operand bits do not toggle, i.e. with the power the random operands draw taken away.
    with torch.no_grad():
        xq0, sx0 = kernels.rotate_quant(x, GROUP)
        u0 = kernels.lowrank_down(x, layer.down.weight)
        xq0.zero_()
        w0 = torch.zeros_like(layer.qweight)
        for _ in range(2):
            kernels.int8_matmul(xq0, w0, sx0, layer.wscale, u=u0, up=layer.up.weight)
        e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        e[0].record(stream)
        for _ in range(5):
            kernels.int8_matmul(xq0, w0, sx0, layer.wscale, u=u0, up=layer.up.weight)
        e[1].record(stream)
        torch.cuda.synchronize()
        ceil["gemm_zero_operands_TOPS"] = round(ops / (e[0].elapsed_time(e[1]) * 1e-3 / 5) / 1e12, 1)
        del xq0, sx0, u0, w0
    ceil["gemm_frac_of_zero_operands"] = round(gemm_tops / ceil["gemm_zero_operands_TOPS"], 4)
    ceil["rotate_quant_frac_of_copy"] = round(result["rotate_quant_GBs"] / ceil["copy_GBs"], 4)
    ceil["rotate_quant_frac_of_stream"] = round(result["rotate_quant_GBs"] / ceil["stream_r2w1_GBs"], 4)
    ceil["lowrank_down_frac_of_stream"] = round(result["lowrank_down_GBs"] / ceil["stream_read_GBs"], 4)
    result["ceilings"] = ceil
    if not args.no_cpu_baseline:
        del x, layer
        torch.cuda.empty_cache()
        result["cpu_baseline"] = cpu_baseline(torch, args.cpu_rows)
    print(json.dumps(result), flush=True)


# ------------------------------------------------------------------------------------------ supporting workloads


def layer_inputs(torch, dev, m, k, n, rank, bias, outlier_frac, outlier_scale, seed, copies=1):
    """Seeded synthetic inputs in the draw order x, outlier channels, qweight, wscale, down, up, bias; `copies`
    independent weight sets for the same x (so a step can rotate through more weight bytes than the cache holds)."""
    from hyperflow_h3_flash_amd import Int8RotLinear

    gen = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(m, k, device=dev, generator=gen)
    cols = torch.randperm(k, device=dev, generator=gen)[: -(-k * int(outlier_frac * 1000) // 1000)]
    x[:, cols] *= outlier_scale
    x = x.to(torch.bfloat16)
    layers = []
    for _ in range(copies):
        layer = Int8RotLinear(k, n, GROUP, rank=rank, bias=bias).to(dev)
        with torch.no_grad():
            layer.qweight.copy_(torch.randint(-127, 128, (n, k), device=dev, dtype=torch.int8, generator=gen))
            layer.wscale.copy_(torch.rand(n, device=dev, generator=gen) * 9e-3 + 1e-3)
            if rank:
                layer.down.weight.copy_(torch.randn(rank, k, device=dev, generator=gen) * 0.02)
                layer.up.weight.copy_(torch.randn(n, rank, device=dev, generator=gen) * 0.02)
            if bias:
                layer.bias.copy_(torch.randn(n, device=dev, generator=gen) * 0.01)
        layers.append(layer)
    return x, layers


def timed(torch, fn, steps, warmup):
    """Mean wall time per call in seconds, with the device synchronized around the timed calls."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def linear_bytes(m, k, n, rank, bias):
    """Compulsory HBM bytes of one fused linear: x, qweight, wscale, low-rank down and up, bias, output."""
    return 2 * m * k + n * k + 4 * n + 2 * rank * (k + n) + (2 * n if bias else 0) + 2 * m * n


def run_config(torch, config, steps, warmup, rows=None, cpu_rows=2048):
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    base = {"n_gpus": 1, "steps": steps, "warmup": warmup, "dtype": "int8", "data": "synthetic (seeded)",
            "vs_baseline": None}
    if config == 1:
        m, k, n, r = 1024, 3072, 3072, 32
        x, (layer,) = layer_inputs(torch, dev, m, k, n, r, True, 0.01, 20.0, seed=1)
        with torch.no_grad():
            t = timed(torch, lambda: layer(x), steps, warmup)
        # the reference's own CPU-runnable case: its CPU path over all 1024 rows, beside the device figure
        cpu = cpu_baseline(torch, m, seed=1, m=m, k=k, n=n, rank=r, bias=True, outlier_frac=0.01, outlier_scale=20.0)
        yield dict(base, metric="convrot INT8 linear TOPS, M=1024 K=3072 N=3072", unit="TOPS",
                   value=round(2.0 * m * n * k / t / 1e12, 2), ms_per_step=round(t * 1e3, 4), higher_is_better=True,
                   hbm_GBs=round(linear_bytes(m, k, n, r, True) / t / 1e9, 1), cpu_baseline=cpu,
                   config={"workload": "single convrot linear", "M": m, "K": k, "N": n, "group": GROUP,
                           "rank": r, "bias": True})
    elif config in (3, 4, 6):
        if config == 3:
            m, shapes, name = 32768, [(5120, 13824), (13824, 5120)], "FFN up + tanh-GELU + down"
        elif config == 6:
            m, shapes, name = 32768, [(5376, 28672), (14336, 5376)], "gated FFN up + SwiGLU + down"
        else:
            # The 5.2 s clip's block (40320 video + 1024 audio tokens); --rows gives one rank's share of it, e.g.
            # 5168 rows for an 8-way split of the tokens.
            m = rows or 41344
            shapes, name = [(5120, 15360), (5120, 5120), (5120, 13824), (13824, 5120)], "DiT block linears"
        built = [layer_inputs(torch, dev, m, k, n, 64, False, 0.005, 30.0, seed=3 + i) for i, (k, n) in
                 enumerate(shapes)]
        xs = [b[0] for b in built]
        layers = [b[1][0] for b in built]

        def step():
            with torch.no_grad():
                if config in (3, 6):
                    # The up-projection applies the activation in its GEMM epilogue (layers[0].activation).
                    layers[1](layers[0](xs[0]))
                else:
                    for x, layer in zip(xs, layers):
                        layer(x)

        def step_unfused():
            with torch.no_grad():
                h = layers[0](xs[0])
                if config == 3:
                    layers[1](torch.nn.functional.gelu(h, approximate="tanh"))
                else:
                    hidden, gate = h.chunk(2, dim=-1)
                    layers[1](hidden * torch.nn.functional.silu(gate))

        extra = {}
        if config in (3, 6):
            t_unfused = timed(torch, step_unfused, steps, warmup)
            layers[0].activation = "gelu_tanh" if config == 3 else "swiglu"
            extra = {"unfused_ms_per_step": round(t_unfused * 1e3, 4)}
        t = timed(torch, step, steps, warmup)
        ops = sum(2.0 * m * n * k for k, n in shapes)
        cpu = None
        if cpu_rows and config in (3, 4):
            del xs, layers, built
            torch.cuda.empty_cache()
            k0, n0 = shapes[0]
            if config == 3:
                chain = [(shapes[1][0], shapes[1][1], "gelu_tanh")]
            else:
                chain = [(shapes[1][0], shapes[1][1], "x"), (shapes[2][0], shapes[2][1], "x"),
                         (shapes[3][0], shapes[3][1], "x")]
            cpu = cpu_baseline(torch, min(cpu_rows, 2048), seed=3, m=m, k=k0, n=n0, rank=64, chain=chain)
        yield dict(base, metric=f"convrot INT8 {name} TOPS, M={m}", unit="TOPS", value=round(ops / t / 1e12, 2),
                   ms_per_step=round(t * 1e3, 4), higher_is_better=True, cpu_baseline=cpu,
                   pct_of_peak=round(100.0 * ops / t / 1e12 / PEAK_INT8_TOPS, 2), **extra,
                   config={"workload": name, "M": m, "shapes_KN": shapes, "group": GROUP, "rank": 64,
                           "bias": False,
                           "activation": {3: "fused tanh-GELU epilogue", 6: "fused SwiGLU epilogue"}.get(config)})
    elif config == 7:
        m = 37710
        for name, k, n in (("q/k/v", 5376, 7168), ("fused q/k/v", 5376, 21504), ("out", 7168, 5376),
                           ("gated up", 5376, 28672), ("down", 14336, 5376)):
            x, (layer,) = layer_inputs(torch, dev, m, k, n, 64, False, 0.005, 30.0, seed=7)
            with torch.no_grad():
                t = timed(torch, lambda: layer(x), steps, warmup)
            yield dict(base, metric=f"convrot INT8 linear TOPS, model {name} M={m} K={k} N={n}", unit="TOPS",
                       value=round(2.0 * m * n * k / t / 1e12, 2), ms_per_step=round(t * 1e3, 4),
                       higher_is_better=True, pct_of_peak=round(100.0 * 2.0 * m * n * k / t / 1e12 / PEAK_INT8_TOPS, 2),
                       config={"workload": f"model linear ({name})", "M": m, "K": k, "N": n, "group": GROUP,
                               "rank": 64, "bias": False})
            del x, layer
            torch.cuda.empty_cache()
    elif config == 8:
        # The standalone low-rank linear (the model's non-INT8 linears, transformer.py:48-72): y = up(down(x)) in
        # bf16 with a bf16 intermediate. Work 2 M r (K + N); the vendor library's bf16 GEMMs (torch's own
        # up(down(x))) are timed on the same tensors beside it.
        from hyperflow_h3_flash_amd import LowRankLinear

        m = 37710
        gen = torch.Generator(device=dev).manual_seed(8)
        for k, n in ((5376, 7168), (14336, 5376)):
            x = torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16)
            for r in (64, 256, 512):
                layer = LowRankLinear(k, n, r).to(dev).to(torch.bfloat16)
                with torch.no_grad():
                    layer.down.weight.copy_(torch.randn(r, k, device=dev, generator=gen) * 0.02)
                    layer.up.weight.copy_(torch.randn(n, r, device=dev, generator=gen) * 0.02)
                    # The two run in alternation over three rounds and each reports its median round: these
                    # memory-bound layers move by 10-25 % with the clock state (the first calls of a process, long
                    # back-to-back runs), and timing one after the other would hand that drift to one side.
                    ours, vendor = [], []
                    for _ in range(3):
                        ours.append(timed(torch, lambda: layer(x), steps, warmup))
                        vendor.append(timed(torch, lambda: layer.up(layer.down(x)), steps, warmup))
                    t, t_vendor = sorted(ours)[1], sorted(vendor)[1]
                flops = 2.0 * m * r * (k + n)
                nbytes = 2 * m * k + 2 * r * (k + n) + 4 * m * r + 2 * m * n
                yield dict(base, dtype="bf16", metric=f"low-rank linear TFLOP/s, M={m} K={k} N={n} rank {r}",
                           unit="TFLOP/s", value=round(flops / t / 1e12, 1), ms_per_step=round(t * 1e3, 4),
                           higher_is_better=True, hbm_GBs=round(nbytes / t / 1e9, 1),
                           vendor_ms=round(t_vendor * 1e3, 4),
                           config={"workload": "standalone low-rank linear up(down(x))", "M": m, "K": k, "N": n,
                                   "rank": r})
                del layer
            del x
            torch.cuda.empty_cache()
    else:
        k = 5120
        for m in (64, 256, 1024) if rows is None else (rows,):
            for n in (5120, 30720):
                copies = max(1, -(-(600 << 20) // (n * k)))  # > 600 MB of weights per pass through the copies
                x, layers = layer_inputs(torch, dev, m, k, n, 32, False, 0.005, 30.0, seed=5, copies=copies)
                # Few rows: the host's per-call work would dominate, so one pass over the weight copies is captured
                # in a HIP graph (as a serving loop would run it) and replayed.
                with torch.no_grad():
                    for layer in layers:
                        layer(x)
                    torch.cuda.synchronize()
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph):
                        for layer in layers:
                            layer(x)
                t = timed(torch, graph.replay, steps, warmup) / copies
                nbytes = linear_bytes(m, k, n, 32, False)
                del graph
                cpu = cpu_baseline(torch, m, seed=5, m=m, k=k, n=n, rank=32) if cpu_rows else None
                yield dict(base, metric=f"convrot INT8 linear HBM GB/s, M={m} K={k} N={n}", unit="GB/s",
                           value=round(nbytes / t / 1e9, 1), ms_per_step=round(t * 1e3, 4), higher_is_better=True,
                           pct_of_hbm_peak=round(100.0 * nbytes / t / 1e9 / PEAK_HBM_GBS, 2),
                           tops=round(2.0 * m * n * k / t / 1e12, 2), cpu_baseline=cpu,
                           config={"workload": "small-M convrot linear", "M": m, "K": k, "N": n, "group": GROUP,
                                   "rank": 32, "bias": False, "weight_copies": copies})
                del x, layers
                torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
