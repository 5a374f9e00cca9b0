"""Benchmark of the quantized linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]

Headline workload (one JSON line on stdout): the W8A8 QuantLinear forward with ConvRot at the
Wan-14B FFN up-projection shape -- x [32760, 5120] bf16 (N(0,1), 1% of channels x20) ->
fused rotate + per-token int8 quantize -> int8 MFMA GEMM with the dequant + bias epilogue ->
y [32760, 13824] bf16.  A step is one forward of the module (both kernels); `value` is
2*M*N*K / step time in TOPS with all inputs resident in HBM.

`roofline` is the int8 GEMM kernel (the dominant one): algorithmic ops per launch divided by
its average launch time, timed with HIP events on its stream around a loop of back-to-back
launches on the headline's quantized input.  `cpu_baseline` is the reference's own CPU path for
the same layer -- QuantLinear's dequantize branch: dequantize_rows (q * s, ConvRot inverse) and
F.linear in bf16 on torch-CPU (powershard/quant_linear.py:219-220, operations.py:84-93) -- on a
bounded row sample, on all of this process's CPU threads and on one, with the int8 weight-only
(1024 x 5120 -> 5120) and uint4 g128 (512 x 5120 -> 25600) layers and one Wan-14B block (x40,
derived) beside it and the C oracle's quantized forward as a second figure.

`extra` carries the other shapes, each with a sampled-row check against the oracle: the int4
(W4A16) text-encoder MLP at M=512 with an M sweep, the fp8 QKV projection, the int8 weight-only
layer, the Wan-14B FFN with its GELU in the up-projection's epilogue against the unfused reference
sequence, the MiniMax-H3 MLP with its SiLU gate in fc1's epilogue (fp16, M=8192) against its
reference sequence, the 8-way token shard's per-GPU share (M=4095), and the 40-block Wan-14B
linear stack.
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "comfyui-powershard_amd"))
sys.path.insert(0, ROOT)

METRIC = "W8A8 GEMM TOPS (% int8 MFMA peak) + int4 GEMM HBM GB/s; Wan-14B block ms"
PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA, TOPS
PEAK_FP8_TFLOPS = 5000.0     # dense fp8
PEAK_BF16_TFLOPS = 2500.0    # dense bf16
PEAK_HBM_GBS = 8000.0        # HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # ~60 ms of warm-up at the headline shape: the GPU's clock ramps over the first ~30 launches
    # after an idle spell (2.4 ms -> 1.75 ms per GEMM launch), and a serving loop runs at the
    # settled clock
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--no-extra", action="store_true", help="headline workload only")
    ap.add_argument("--extras", default="", help="comma-separated subset of the extra workloads to run "
                    "(int4_w4a16, fp8, w8a16, wan_ffn_gelu, h3_mlp_silu_gate, shard_m4095, wan14b_stack; "
                    "gemm_i8_8wave, the int8 GEMM's 8-wave comparison schedule, only when named); default all")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=3.0,
                    help="target time of each timed CPU baseline sample (about ten samples in all)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain elementwise copy of 1 GiB (3 launches), the reference point that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    return ap.parse_args()


# ---------------------------------------------------------------------- inputs
def gen(seed):
    import torch
    return torch.Generator(device="cuda").manual_seed(seed)


def activations(M, K, sid, outlier_scale=20.0, student_t=False, dev="cuda"):
    """bf16 [M, K]: N(0,1) (or Student-t, df=3) with 1% of channels (seeded pick) scaled; `sid`
    offsets the seeds so that each workload draws its own synthetic inputs."""
    import torch
    g = gen(2000 + sid)
    x = torch.randn(M, K, generator=g, device=dev)
    if student_t:
        chi = torch.zeros_like(x)
        for _ in range(3):
            chi += torch.randn(M, K, generator=g, device=dev) ** 2
        x /= (chi / 3).sqrt()
    gp = torch.Generator().manual_seed(4000 + sid)
    idx = torch.randperm(K, generator=gp)[: int(0.01 * K)].to(dev)
    x[:, idx] *= outlier_scale
    return x.to(torch.bfloat16)


def quant_layer(K, N, weight_format, sid, seed=None, opts=None, dev="cuda", dtype=None):
    """A QuantLinear installed and filled through the package's own install/pack path (compute
    dtype bf16 unless given)."""
    import torch
    from torch import nn
    from powershard_amd.quant_linear import install_quant_linears, quantized_from_float, pack
    g = gen(1000 + sid if seed is None else seed)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    dtype = dtype or torch.bfloat16
    b = (torch.randn(N, generator=gen(3000 + sid), device=dev) * 0.01).to(dtype)
    with torch.device("meta"):
        net = nn.Sequential(nn.Linear(K, N, dtype=dtype))
    tensors = {"0.weight": {"key": "0.weight", "dtype": "BF16", "shape": [N, K]}}
    install_quant_linears(net, tensors, weight_format, "native", None, dtype, torch.device(dev),
                          quant_options=opts)
    layer = net[0]
    qt = quantized_from_float(w, layer._ps_qplan.fmt, **(opts or {}))
    layer.qbytes = nn.Parameter(pack(qt, layer._ps_qplan, dev), requires_grad=False)
    layer.bias = nn.Parameter(b, requires_grad=False)
    del w
    return layer, qt, b


def fused_vs_reference(got, ref):
    """Errors of a fused MLP against the reference sequence on the same modules: max and RMS of the
    difference over the output RMS, and whether every element is within max(1e-2 RMS, one bf16 ulp
    of the reference value).  A hidden element one ulp away can move its row's per-token scale in
    the down projection, which shifts that row by up to a quantization step: on heavy-tailed rows
    that exceeds 1e-2 RMS only where one ulp of the output itself does."""
    import torch
    got, ref = got.float(), ref.float()
    rms = ref.pow(2).mean().sqrt()
    err = (got - ref).abs()
    ulp = torch.pow(2.0, torch.floor(torch.log2(ref.abs().clamp(min=1e-30))) - 7)
    bound = torch.maximum(1e-2 * rms, ulp)
    return dict(max_err_over_rms=(err.max() / rms).item(), rms_err_over_rms=(err.pow(2).mean().sqrt() / rms).item(),
                within_bar=bool((err <= bound).all().item()), frac_over_1e2_rms=(err > 1e-2 * rms).double().mean().item())


# ---------------------------------------------------------------------- timing
def timed_steps(step, steps, warmup):
    """(ms per step from events around the whole loop, {kernel: mean ms per launch})."""
    import torch
    from powershard_amd import ops
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with ops.kernel_timer() as ev:
        start.record()
        for _ in range(steps):
            step()
        end.record()
        torch.cuda.synchronize()
    total = start.elapsed_time(end)
    per = {k: sum(v) / len(v) for k, v in ops.kernel_times_ms(ev).items()}
    return total / steps, per


def untimed_kernel_ms(step, steps, warmup):
    """Same as timed_steps without per-launch events (pure step time)."""
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


# -------------------------------------------------------------------- workloads
def headline(args):
    import torch
    from powershard_amd import ops
    M, K, N = 32760, 5120, 13824
    sid = 1
    log(f"[bench] headline W8A8+ConvRot M={M} K={K} N={N}: building inputs")
    x = activations(M, K, sid)
    layer, qt, b = quant_layer(K, N, "int8", sid, opts={"convrot": True, "convrot_groupsize": 256})
    with torch.no_grad():
        y = layer(x)
    if not layer._ps_native:
        raise RuntimeError("native path fell back to dequantize")
    # each kernel alone, back to back on the same stream: events around the loop, not per launch.
    # These run first: the shader clock ramps up over the first ~30 GEMM launches after an idle
    # spell, and these loops (untimed for the headline) leave it settled, as in a serving loop,
    # whatever warm-up count the headline is given.
    qx, sx = ops.quantize_rows(x, rot_group=256)
    wq, ws = qt._qdata, qt._params.scale
    gemm_ms = untimed_kernel_ms(lambda: ops.gemm_i8(qx, sx, wq, ws, b), max(args.steps, 20), 10)
    quant_ms = untimed_kernel_ms(lambda: ops.quantize_rows(x, rot_group=256), max(args.steps, 20), 3)
    log(f"[bench] headline: warmup {args.warmup}, timing {args.steps} steps")

    def step():
        with torch.no_grad():
            layer(x)
    ms = untimed_kernel_ms(step, args.steps, args.warmup)
    ops_per_step = 2.0 * M * N * K
    tops = ops_per_step / (ms * 1e-3) / 1e12
    gemm_tops = ops_per_step / (gemm_ms * 1e-3) / 1e12
    quant_bytes = M * K * 2 + M * K + M * 4
    res = dict(M=M, N=N, K=K, ms_per_step=ms, tops=tops, gemm_ms=gemm_ms, gemm_tops=gemm_tops, quant_ms=quant_ms,
               quant_gbs=quant_bytes / (quant_ms * 1e-3) / 1e9, quant_bytes=quant_bytes)
    log(f"[bench] headline: {ms:.3f} ms/step, {tops:.1f} TOPS; gemm {gemm_ms:.3f} ms = {gemm_tops:.1f} TOPS "
        f"({100 * gemm_tops / PEAK_INT8_TOPS:.1f}% of int8 peak); quant {quant_ms * 1e3:.1f} us = "
        f"{res['quant_gbs']:.0f} GB/s")
    # parity rows: the first 64, 128 spread over the middle, and the last 64 (the partial last tile)
    idx = sample_rows(M, 256, 5000 + sid)
    sample = dict(x=x[:4096].cpu(), qdata=qt._qdata.cpu(), scale=qt._params.scale.cpu(), bias=b.cpu(),
                  rows=idx, x_rows=x[idx.to(x.device)].cpu(), y_rows=y[idx.to(y.device)].cpu(), M=M)
    del layer, qt, x, y, qx, sx
    torch.cuda.empty_cache()
    return res, sample


def sample_rows(M, n, seed):
    """n row indices: the first and last quarter-n rows (the edge tiles) and the rest spread between."""
    import torch
    if M <= n:
        return torch.arange(M)
    e = n // 4
    g = torch.Generator().manual_seed(seed)
    mid = torch.randperm(M - 2 * e, generator=g)[: n - 2 * e] + e
    return torch.cat([torch.arange(e), mid.sort().values, torch.arange(M - e, M)])


def check_headline_parity(sample):
    """Bit-exact check of 256 sampled rows of the headline output (first, spread, last -- the last
    ones in the partial tile) against the oracle (rotate + quantize, int32 GEMM, epilogue)."""
    import torch
    import oracle
    qa, sa = oracle.quantize_rows_i8(sample["x_rows"], 256)
    ref = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, sample["qdata"]), sa, sample["scale"], sample["bias"])
    got = sample["y_rows"]
    same = bool(torch.equal(got.view(torch.int16), ref.view(torch.int16)))
    err = (got.float() - ref.float()).abs().max().item()
    rms = ref.float().pow(2).mean().sqrt().item()
    return dict(rows_checked=int(sample["rows"].numel()), bitexact=same, max_abs_err_over_rms=err / rms)


def within_bar(got, ref):
    """Sampled-row check of an fp32-accumulating path: every element within max(1e-2 rms, one bf16
    ulp of the reference value) -- the ulp covers rounding ties of two fp32 sums at large |y|."""
    import torch
    got, ref = got.float(), ref.float()
    rms = ref.pow(2).mean().sqrt()
    err = (got - ref).abs()
    ulp = torch.pow(2.0, torch.floor(torch.log2(ref.abs().clamp(min=1e-30))) - 7)
    return dict(rows_checked=int(got.shape[0]), within_bar=bool((err <= torch.maximum(1e-2 * rms, ulp)).all()),
                max_abs_err_over_rms=(err.max() / rms).item())


PROFILE = os.path.join(ROOT, "profiles", "gemm_i8_w8a8_convrot_m32760_n13824_k5120.md")


def profiled_traffic():
    """HBM-side bytes per launch of the headline GEMM: FETCH_SIZE and WRITE_SIZE (rocprofv3 --pmc,
    one counter per run) scaled by their copy-kernel calibration factors, as recorded in the
    kernel's profile summary.  None when the summary is absent."""
    try:
        text = open(PROFILE).read()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        d = json.loads(block)
        return dict(bytes=int(d["read_bytes"] + d["write_bytes"]),
                    source=f"profiles/{os.path.basename(PROFILE)}: FETCH_SIZE x{d['fetch_factor']} "
                           f"+ WRITE_SIZE x{d['write_factor']} per launch (L2 <-> fabric bytes)")
    except (OSError, IndexError, KeyError, ValueError):
        return None


# ------------------------------------------------------------------ CPU baseline
def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _seconds(fn):
    t0 = time.perf_counter()
    out = fn()
    return time.perf_counter() - t0, out


def reference_cpu_forward(dequant, x_rows, M, bias, target_s):
    """Time the reference's dequantize-branch forward on the CPU: the per-call dequantization of
    the whole weight (independent of M) and the bf16 F.linear on a row sample grown until it takes
    about target_s / 3; the M-row forward is projected as t_dequant + t_linear * M / rows."""
    import torch
    t_deq, w = _seconds(dequant)
    N, K = w.shape
    torch.nn.functional.linear(x_rows[:4], w, bias)          # kernel selection / first-call work
    rows = 4
    while True:
        t_lin, _ = _seconds(lambda: torch.nn.functional.linear(x_rows[:rows], w, bias))
        if t_lin * 3 > target_s or rows >= min(M, x_rows.shape[0]):
            break
        rows = min(rows * 4, M, x_rows.shape[0])
    t_full = t_deq + t_lin * M / rows
    return dict(tops=2.0 * M * N * K / t_full / 1e12, forward_s=t_full, dequant_s=t_deq, linear_rows=rows,
                linear_s=t_lin)


def _convrot_dequant(q, s, g):
    import oracle
    import torch
    return lambda: oracle.dequantize_rows(q, s, g > 0, g, torch.bfloat16)


def _rowwise_dequant(q, s):
    import torch
    return lambda: (q.float() * s.float().reshape(-1, 1)).to(torch.bfloat16)


def _uint4_dequant(wq, s, z, g):
    """w = (q - z) s per (row, group), low nibble = even k, then bf16: torch ops on the CPU."""
    import torch

    def run():
        q = torch.stack([wq & 15, wq >> 4], -1).reshape(wq.shape[0], -1).float()
        zz = z.float().repeat_interleave(g, 1)
        ss = s.float().repeat_interleave(g, 1)
        return ((q - zz) * ss).to(torch.bfloat16)
    return run


def cpu_inputs(sample):
    """CPU copies of the int8 weight-only, uint4 and one-Wan-block layers, built on the GPU with the seeds of
    their GPU workloads, and their activation rows."""
    import torch
    c = {}
    layer, qt, b = quant_layer(5120, 5120, "int8", 0)
    c["int8_wonly"] = dict(q=qt._qdata.cpu(), s=qt._params.scale.cpu(), b=b.cpu(),
                           x=activations(1024, 5120, 0, outlier_scale=1.0).cpu())
    layer, qt, b = quant_layer(5120, 25600, "int4", 2, seed=1002, opts={"group_size": 128})
    p = qt._params
    c["uint4"] = dict(q=qt._qdata.cpu(), s=p.scale.cpu(), z=p.zero.cpu(), b=b.cpu(),
                   x=activations(512, 5120, 2, outlier_scale=1.0).cpu())
    opts = {"convrot": True, "convrot_groupsize": 256}
    blk = []
    for i, (k_, n_) in enumerate(((5120, 5120),) * 4 + ((5120, 13824), (13824, 5120))):
        layer, qt, b = quant_layer(k_, n_, "int8", 4, seed=1004 + i + 1, opts=opts)
        blk.append(dict(q=qt._qdata.cpu(), s=qt._params.scale.cpu(), b=b.cpu()))
    c["wan_block"] = dict(layers=blk, x=activations(256, 5120, 4, outlier_scale=50.0, student_t=True).cpu(),
                   h=activations(256, 13824, 104, outlier_scale=50.0, student_t=True).cpu())
    del layer, qt
    torch.cuda.empty_cache()
    return c


def cpu_baseline(sample, inputs, target_s):
    """The reference's CPU path (QuantLinear dequantize branch on torch-CPU) for the headline layer on
    all threads and on one, the int8 weight-only and uint4 layers and one Wan-14B block (x40,
    derived), and the C
    oracle's quantized W8A8 forward as a second figure."""
    import torch
    import oracle
    threads = torch.get_num_threads()
    M, (N, K) = sample["M"], sample["qdata"].shape
    q, s, b, x = sample["qdata"], sample["scale"], sample["bias"], sample["x"]
    head = reference_cpu_forward(_convrot_dequant(q, s, 256), x, M, b, target_s)
    log(f"[bench] cpu reference path, {threads} threads: {head['tops'] * 1e3:.1f} GOPS (dequant "
        f"{head['dequant_s']:.2f} s, linear {head['linear_rows']} rows {head['linear_s']:.2f} s)")
    torch.set_num_threads(1)
    try:
        one = reference_cpu_forward(_convrot_dequant(q, s, 256), x, M, b, target_s)
    finally:
        torch.set_num_threads(threads)
    log(f"[bench] cpu reference path, 1 thread: {one['tops'] * 1e3:.1f} GOPS")
    configs = {}
    wonly = inputs["int8_wonly"]
    configs["int8_weight_only_1024x5120x5120"] = reference_cpu_forward(
        _rowwise_dequant(wonly["q"], wonly["s"]), wonly["x"], 1024, wonly["b"], target_s)
    u4 = inputs["uint4"]
    configs["uint4_g128_512x5120x25600"] = reference_cpu_forward(
        _uint4_dequant(u4["q"], u4["s"], u4["z"], 128), u4["x"], 512, u4["b"], target_s)
    blk = inputs["wan_block"]
    block_s, block_ops = 0.0, 0.0
    for i, lay in enumerate(blk["layers"]):
        xr = blk["h"] if i == 5 else blk["x"]
        r = reference_cpu_forward(_convrot_dequant(lay["q"], lay["s"], 256), xr, 32760, lay["b"], target_s / 3)
        block_s += r["forward_s"]
        block_ops += 2.0 * 32760 * lay["q"].shape[0] * lay["q"].shape[1]
    configs["wan14b_40_blocks_derived"] = dict(block_s=block_s, total_s=40 * block_s,
                                                  tops=block_ops / block_s / 1e12,
                                                  note="one block timed (6 layers, row samples), x40")
    for k, v in configs.items():
        log(f"[bench] cpu reference path {k}: {v['tops'] * 1e3:.1f} GOPS")
    # the oracle's quantized forward (rotate + quantize, int32 GEMM, epilogue) in C with OpenMP
    def oracle_forward(rows):
        qa, sa = oracle.quantize_rows_i8(x[:rows], 256)
        return oracle.epilogue_i32(oracle.gemm_i8_i32(qa, q), sa, s, b)
    rows = 8
    while True:
        t, _ = _seconds(lambda: oracle_forward(rows))
        if t * 3 > target_s or rows >= x.shape[0]:
            break
        rows = min(x.shape[0], rows * 4)
    orc = dict(tops=2.0 * rows * N * K / t / 1e12, rows=rows, seconds=t, threads=oracle.num_threads())
    return dict(value=head["tops"], unit="TOPS", cores=threads, kind="port", cpu_model=cpu_model(),
                algorithm="the reference's CPU path: dequantize_rows (q*s, ConvRot inverse) + bf16 F.linear "
                          "(powershard/quant_linear.py:219-220, operations.py:84-93) on torch-CPU",
                sample=f"headline layer {M}x{K}->{N}: dequantization of the whole weight timed once "
                       f"({head['dequant_s']:.2f} s), F.linear on {head['linear_rows']} rows "
                       f"({head['linear_s']:.2f} s), projected to M={M}; same synthetic inputs as the GPU run",
                detail=head, single_thread=dict(value=one["tops"], unit="TOPS", detail=one), configs=configs,
                oracle_w8a8=dict(value=orc["tops"], unit="TOPS", rows=orc["rows"], seconds=orc["seconds"],
                                 threads=orc["threads"],
                                 note="C oracle: rotate+quantize, int32 GEMM, epilogue (the quantized reference)"))


def extra_int4(args):
    """W4A16 uint4 g128 Qwen3-VL-32B text-encoder MLP, K=5120 -> N=25600; M sweep.  Weights rotate
    over 12 distinct copies (12 x 69.6 MB = 835 MB, over three times the 256 MB Infinity Cache), so
    each launch streams its weights from HBM; each M is timed as a loop of 100 back-to-back kernel
    launches with events around the loop, after 400 untimed ones.  M = 1 and M = 512 are checked on
    sampled rows."""
    import torch
    import oracle
    from powershard_amd import ops
    K, N, sid, copies = 5120, 25600, 2, 12
    layers = [quant_layer(K, N, "int4", sid, seed=1000 + sid + 17 * i, opts={"group_size": 128}) for i in range(copies)]
    ws = [(qt._qdata, qt._params.scale, qt._params.zero, b) for _, qt, b in layers]
    out, parity = {}, {}
    for M in (1, 16, 32, 64, 128, 256, 512):
        x = activations(M, K, sid, outlier_scale=1.0)
        it = [0]

        def step():
            q, sc, z, b = ws[it[0] % copies]
            ops.gemm_w4a16(x, q, sc, z, 128, b)
            it[0] += 1
        # a serving loop's steady state: the shader clock of these short launches settles over
        # ~10 ms of back-to-back launches (M=1: 26 us over the first 500 launches, 24 us after)
        kms = untimed_kernel_ms(step, max(args.steps, 100), max(args.warmup, 400))
        wbytes = N * K // 2 + 2 * 2 * N * (K // 128)
        algo_bytes = wbytes + M * K * 2 + M * N * 2
        flops = 2.0 * M * N * K
        out[M] = dict(kernel_ms=kms, hbm_gbs=algo_bytes / (kms * 1e-3) / 1e9,
                      hbm_frac=algo_bytes / (kms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                      tflops=flops / (kms * 1e-3) / 1e12, bf16_mfma_frac=flops / (kms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS)
        log(f"[bench] int4 M={M}: {kms * 1e3:.1f} us, {out[M]['hbm_gbs']:.0f} GB/s, {out[M]['tflops']:.1f} TFLOP/s")
        if M in (1, 512):
            layer, qt, b = layers[0]
            with torch.no_grad():
                y = layer(x)
            rows = sample_rows(M, 64, 6000 + M)
            p = qt._params
            wd = oracle.dequant_uint4(qt._qdata.cpu(), p.scale.cpu(), p.zero.cpu(), 128)
            ref = oracle.gemm_wonly(x[rows.to(x.device)].cpu(), wd, None, b.cpu(), out_dtype=torch.float32)
            parity[M] = within_bar(y[rows.to(y.device)].cpu(), ref)
            log(f"[bench] int4 M={M} parity: {parity[M]}")
    del layers, ws
    torch.cuda.empty_cache()
    return dict(workload="W4A16 uint4 asym g128, K=5120->N=25600", weight_copies=copies, sweep=out, parity=parity)


def extra_fp8(args):
    import torch
    import oracle
    M, K, N, sid = 32760, 5120, 15360, 3
    x = activations(M, K, sid, outlier_scale=1.0)
    layer, qt, b = quant_layer(K, N, "fp8", sid)

    def step():
        with torch.no_grad():
            layer(x)
    ms = untimed_kernel_ms(step, args.steps, args.warmup)
    from powershard_amd import ops
    qx, sx = ops.quantize_rows(x, fp8=True)
    gemm_ms = untimed_kernel_ms(lambda: ops.gemm_fp8(qx, sx, qt._qdata, qt._params.scale, b), args.steps, 3)
    quant_ms = untimed_kernel_ms(lambda: ops.quantize_rows(x, fp8=True), args.steps, 3)
    flops = 2.0 * M * N * K
    res = dict(workload="fp8 e4m3 per-token x per-tensor, Wan-14B QKV 5120->15360, M=32760", ms_per_step=ms,
               tflops=flops / (ms * 1e-3) / 1e12, gemm_ms=gemm_ms, gemm_tflops=flops / (gemm_ms * 1e-3) / 1e12,
               gemm_frac=flops / (gemm_ms * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, quant_ms=quant_ms)
    with torch.no_grad():
        y = layer(x)
    rows = sample_rows(M, 64, 6003)
    xr = x[rows.to(x.device)].cpu()
    qa, sa = oracle.quantize_rows_fp8(xr)
    ref = oracle.gemm_fp8(qa, sa, qt._qdata.cpu().view(torch.uint8), qt._params.scale.cpu(), b.cpu(),
                          out_dtype=torch.float32)
    res["parity"] = within_bar(y[rows.to(y.device)].cpu(), ref)
    log(f"[bench] fp8: {ms:.3f} ms/step, gemm {res['gemm_tflops']:.0f} TFLOP/s ({100 * res['gemm_frac']:.1f}%); "
        f"parity {res['parity']}")
    del layer, x, qx, sx, y
    torch.cuda.empty_cache()
    return res


def extra_wan_stack(args):
    """40 Wan-14B blocks of W8A8+ConvRot linears at M=32760 (q, k, v, o, ffn up, ffn down);
    heavy-tailed inputs (Student-t df=3, 1% channels x50); random-init int8 weights per block.
    Four activation quantizations per block: q, k and v share theirs (reuse_quantized_inputs)."""
    import torch
    M, D, F, sid = 32760, 5120, 13824, 4
    opts = {"convrot": True, "convrot_groupsize": 256}
    blocks = []
    for blk in range(40):
        seed = 1000 + sid + 1000 * blk
        q = quant_layer(D, D, "int8", sid, seed=seed + 1, opts=opts)[0]
        k = quant_layer(D, D, "int8", sid, seed=seed + 2, opts=opts)[0]
        v = quant_layer(D, D, "int8", sid, seed=seed + 3, opts=opts)[0]
        o = quant_layer(D, D, "int8", sid, seed=seed + 4, opts=opts)[0]
        up = quant_layer(D, F, "int8", sid, seed=seed + 5, opts=opts)[0]
        down = quant_layer(F, D, "int8", sid, seed=seed + 6, opts=opts)[0]
        blocks.append((q, k, v, o, up, down))
    x = activations(M, D, sid, outlier_scale=50.0, student_t=True)
    h = activations(M, F, sid + 100, outlier_scale=50.0, student_t=True)

    from powershard_amd.quant_linear import reuse_quantized_inputs

    def step():
        with torch.no_grad():
            for q, k, v, o, up, down in blocks:
                with reuse_quantized_inputs():   # q, k, v quantize their common input once
                    q(x); k(x); v(x)
                o(x); up(x); down(h)
    steps = max(2, min(args.steps, 3))
    ms, per = timed_steps(step, steps, 1)
    ops_per_block = 2.0 * M * (4 * D * D + 2 * D * F)
    res = dict(workload="40 Wan-14B blocks (q,k,v,o 5120^2; ffn 5120<->13824) W8A8+ConvRot, M=32760",
               ms_total=ms, ms_per_block=ms / 40, tops=40 * ops_per_block / (ms * 1e-3) / 1e12,
               frac_int8_peak=40 * ops_per_block / (ms * 1e-3) / 1e12 / PEAK_INT8_TOPS,
               quant_ms_mean=per["quantize_rows_i8"], gemm_ms_mean=per["gemm_i8"])
    # parity: block 0's FFN up projection on the heavy-tailed input, 64 sampled rows, bit-exact
    import oracle
    from powershard_amd import quant_linear as ql
    up = blocks[0][4]
    with torch.no_grad():
        y = up(x)
    qt0 = ql.unpack(up.qbytes, up._ps_qplan)
    rows = sample_rows(M, 64, 6004)
    qa, sa = oracle.quantize_rows_i8(x[rows.to(x.device)].cpu(), 256)
    ref = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qt0._qdata.cpu()), sa, qt0._params.scale.cpu(), up.bias.cpu())
    res["parity"] = dict(rows_checked=64, layer="block 0 ffn up",
                         bitexact=bool(torch.equal(y[rows.to(y.device)].cpu().view(torch.int16), ref.view(torch.int16))))
    log(f"[bench] wan stack: {ms:.1f} ms total, {ms / 40:.2f} ms/block, {res['tops']:.0f} TOPS; parity {res['parity']}")
    del blocks, x, h, y
    torch.cuda.empty_cache()
    return res


def extra_ffn(args):
    """Wan-14B FFN (powershard/wan_model.py:621-628) at M=32760: up 5120->13824, GELU(tanh), down
    13824->5120, W8A8+ConvRot.  The reference sequence F.gelu(up(x).float()) -> down (fp32 hidden,
    cast to bf16 by down) against the GELU in the up-projection's epilogue (up.forward_act)."""
    import torch
    import torch.nn.functional as Fn
    M, D, F, sid = 32760, 5120, 13824, 4
    opts = {"convrot": True, "convrot_groupsize": 256}
    up = quant_layer(D, F, "int8", sid, seed=1000 + sid + 5, opts=opts)[0]
    down = quant_layer(F, D, "int8", sid, seed=1000 + sid + 6, opts=opts)[0]
    x = activations(M, D, sid, outlier_scale=50.0, student_t=True)
    steps = max(3, min(args.steps, 10))
    res = {"workload": "Wan-14B FFN up 5120->13824, GELU(tanh), down 13824->5120, W8A8+ConvRot, M=32760"}
    with torch.no_grad():
        res["unfused_ms"] = untimed_kernel_ms(lambda: down(Fn.gelu(up(x).float(), approximate="tanh")), steps, 1)
        res["fused_ms"] = untimed_kernel_ms(lambda: down(up.forward_act(x)), steps, 1)
        # the epilogue's cost: the up-projection alone, without and with the GELU
        res["up_ms"] = untimed_kernel_ms(lambda: up(x), steps, 1)
        res["up_gelu_ms"] = untimed_kernel_ms(lambda: up.forward_act(x), steps, 1)
        ref = down(Fn.gelu(up(x).float(), approximate="tanh")).float()
        got = down(up.forward_act(x)).float()
        res.update(fused_vs_reference(got, ref))
    log(f"[bench] wan ffn: unfused {res['unfused_ms']:.3f} ms, fused {res['fused_ms']:.3f} ms; up GEMM "
        f"{res['up_ms']:.3f} ms, with GELU {res['up_gelu_ms']:.3f} ms; max err/rms {res['max_err_over_rms']:.2e}, "
        f"rms err/rms {res['rms_err_over_rms']:.2e}, within max(1e-2 rms, 1 ulp): {res['within_bar']}")
    del up, down, x
    torch.cuda.empty_cache()
    return res


def extra_h3_mlp(args):
    """MiniMax-H3 MLP (powershard/fp16_safe.py:126-172; fc1 28672x5376, fc2 5376x14336 as in the
    reference's int8-ConvRot checkpoint headers) at M=8192 synthetic tokens, fp16 compute
    (h3_quant.py:101-105), W8A8+ConvRot: the reference sequence gate, up = fc1(x).chunk(2, -1);
    fc2(F.silu(gate.float()) * up.float()) against the gate in fc1's epilogue."""
    import torch
    import torch.nn.functional as Fn
    M, D, F, sid = 8192, 5376, 14336, 5
    opts = {"convrot": True, "convrot_groupsize": 256}
    fc1 = quant_layer(D, 2 * F, "int8", sid, seed=5000, opts=opts, dtype=torch.float16)[0]
    fc2 = quant_layer(F, D, "int8", sid, seed=5001, opts=opts, dtype=torch.float16)[0]
    # N(0,1) with 1% of channels x20: fc1's outputs stay well inside fp16 (heavier tails overflow
    # the fp16 hidden of the reference sequence itself)
    x = activations(M, D, sid).to(torch.float16)
    steps = max(3, min(args.steps, 10))

    def unfused():
        gate, up = fc1(x).chunk(2, -1)
        return fc2(Fn.silu(gate.float()) * up.float())
    res = {"workload": "MiniMax-H3 MLP fc1 5376->2x14336, SiLU gate, fc2 14336->5376, W8A8+ConvRot, fp16, M=8192"}
    with torch.no_grad():
        res["unfused_ms"] = untimed_kernel_ms(unfused, steps, 1)
        res["fused_ms"] = untimed_kernel_ms(lambda: fc2(fc1.forward_act(x, "silu_gate")), steps, 1)
        res["fc1_ms"] = untimed_kernel_ms(lambda: fc1(x), steps, 1)
        res["fc1_gate_ms"] = untimed_kernel_ms(lambda: fc1.forward_act(x, "silu_gate"), steps, 1)
        ref = unfused().float()
        got = fc2(fc1.forward_act(x, "silu_gate")).float()
        if not (torch.isfinite(ref).all() and torch.isfinite(got).all()):
            raise RuntimeError("h3 mlp: non-finite outputs")
        res.update(fused_vs_reference(got, ref))
    log(f"[bench] h3 mlp: unfused {res['unfused_ms']:.3f} ms, fused {res['fused_ms']:.3f} ms; fc1 GEMM "
        f"{res['fc1_ms']:.3f} ms, with the gate {res['fc1_gate_ms']:.3f} ms; max err/rms {res['max_err_over_rms']:.2e}, "
        f"rms err/rms {res['rms_err_over_rms']:.2e}, within max(1e-2 rms, 1 ulp): {res['within_bar']}")
    del fc1, fc2, x
    torch.cuda.empty_cache()
    return res


def extra_shard(args):
    """The per-GPU share of the 8-way token-sharded Wan-14B layer (M_local = ceil(32760 / 8) = 4095):
    the headline QuantLinear forward and one Wan block of W8A8+ConvRot linears at that M, to set
    against the single-GPU figures when planning the sharded path (one GPU runs it here)."""
    import torch
    M, D, F, sid = 4095, 5120, 13824, 4
    opts = {"convrot": True, "convrot_groupsize": 256}
    from powershard_amd.quant_linear import reuse_quantized_inputs
    up = quant_layer(D, F, "int8", 1, opts=opts)[0]
    x = activations(M, D, 1)
    steps = max(10, args.steps)
    with torch.no_grad():
        fwd_ms = untimed_kernel_ms(lambda: up(x), steps, 3)
    layers = [quant_layer(D, D, "int8", sid, seed=2000 + i, opts=opts)[0] for i in range(4)]
    down = quant_layer(F, D, "int8", sid, seed=2010, opts=opts)[0]
    xs = activations(M, D, sid, outlier_scale=50.0, student_t=True)
    h = activations(M, F, sid + 100, outlier_scale=50.0, student_t=True)
    q, k, v, o = layers

    def block():
        with torch.no_grad():
            with reuse_quantized_inputs():
                q(xs); k(xs); v(xs)
            o(xs); up(xs); down(h)
    block_ms = untimed_kernel_ms(block, steps, 2)
    ops_block = 2.0 * M * (4 * D * D + 2 * D * F)
    res = dict(workload="8-way token shard of Wan-14B at M_local=4095: FFN up forward and one block (W8A8+ConvRot)",
               up_forward_ms=fwd_ms, up_forward_tops=2.0 * M * D * F / (fwd_ms * 1e-3) / 1e12,
               block_ms=block_ms, block_tops=ops_block / (block_ms * 1e-3) / 1e12)
    log(f"[bench] shard M=4095: up forward {fwd_ms:.3f} ms ({res['up_forward_tops']:.0f} TOPS), "
        f"block {block_ms:.3f} ms ({res['block_tops']:.0f} TOPS)")
    del layers, up, down, x, xs, h
    torch.cuda.empty_cache()
    return res


def extra_w8a16(args):
    import torch
    M, K, N, sid = 1024, 5120, 5120, 0
    from powershard_amd import ops
    x = activations(M, K, sid, outlier_scale=1.0)
    layer, qt, b = quant_layer(K, N, "int8", sid)
    q, s = qt._qdata, qt._params.scale

    def step():
        ops.gemm_w8a16(x, q, s, b)
    kms = untimed_kernel_ms(step, max(args.steps, 20), args.warmup)
    flops = 2.0 * M * N * K
    res = dict(workload="int8 weight-only (W8A16) 1024x5120x5120", kernel_ms=kms, tflops=flops / (kms * 1e-3) / 1e12)
    import oracle
    y = ops.gemm_w8a16(x, q, s, b)
    rows = sample_rows(M, 64, 6000)
    ref = oracle.gemm_wonly(x[rows.to(x.device)].cpu(), q.cpu().to(torch.bfloat16), s.cpu(), b.cpu(),
                            out_dtype=torch.float32)
    res["parity"] = within_bar(y[rows.to(y.device)].cpu(), ref)
    log(f"[bench] w8a16: {kms * 1e3:.1f} us, {res['tflops']:.0f} TFLOP/s; parity {res['parity']}")
    # Int8Linear (powershard/operations.py:96-132) with ConvRot storage on the same shape: the kernel
    # path (rotate + W8A16) against the reference's 256-row tile dequantization + F.linear
    from powershard_amd.operations import Int8Linear
    layers = []
    for native in (True, False):
        lin = Int8Linear(torch.nn.Linear(K, N, bias=True), dict(convrot=True, group_size=256), rows=256)
        lin = lin.to_empty(device="cuda")
        lin.weight.data.copy_(q)
        lin.weight_scale.data.copy_(s.reshape(-1, 1))
        lin.bias = torch.nn.Parameter(b.half(), requires_grad=False)
        lin._ps_native = native
        layers.append(lin)
    xh = x.half()
    for name, lin in zip(("int8linear_kernel_ms", "int8linear_tiles_ms"), layers):
        res[name] = untimed_kernel_ms(lambda: lin(xh), max(args.steps, 20), args.warmup)
    res["int8linear_workload"] = "Int8Linear ConvRot g=256, fp16, 1024x5120x5120: rotate + W8A16 vs 256-row tiles"
    log(f"[bench] Int8Linear: kernels {res['int8linear_kernel_ms'] * 1e3:.1f} us, "
        f"tile dequant {res['int8linear_tiles_ms'] * 1e3:.1f} us")
    return res


def extra_8wave(args):
    """The int8 GEMM's 8-wave comparison schedule (psq_gemm_i8_8wave: two waves per SIMD, 128 x 64
    wave tiles, the same ring) against the kernel in use (psq_gemm_i8), bf16 output with a bias, on
    the c1 and c4-down GEMMs: launches of the two alternate in rounds (10 untimed + 20 timed each,
    three rounds, the fastest round kept), outputs compared bit for bit.  Run only when named."""
    import ctypes
    import torch
    from powershard_amd import _native
    lib = _native.lib()
    res = {}
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    for tag, (M, N, K) in (("c1_ffn_up", (32760, 13824, 5120)), ("c4_ffn_down", (32760, 5120, 13824))):
        g = gen(8100 + N)
        a = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
        w = torch.randint(-127, 128, (N, K), generator=g, device="cuda", dtype=torch.int8)
        sa = torch.rand(M, generator=g, device="cuda") * 0.01 + 1e-3
        sw = torch.rand(N, generator=g, device="cuda") * 1e-3 + 1e-5
        b = (torch.randn(N, generator=g, device="cuda") * 0.1).to(torch.bfloat16)
        ys = {n: torch.empty(M, N, dtype=torch.bfloat16, device="cuda") for n in ("gemm_i8", "gemm_i8_8wave")}
        fns = {"gemm_i8": lib.psq_gemm_i8, "gemm_i8_8wave": lib.psq_gemm_i8_8wave}

        def run(n):
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            rc = fns[n](P(a), K, P(sa), P(w), K, P(sw), P(b), _native.BF16, P(ys[n]), _native.BF16, N, M, N, K, st)
            if rc != 0:
                raise RuntimeError(_native.last_error())
        times = {n: [] for n in fns}
        for _ in range(3):
            for n in fns:
                times[n].append(untimed_kernel_ms(lambda: run(n), 20, 10))
        same = torch.equal(ys["gemm_i8"].view(torch.int16), ys["gemm_i8_8wave"].view(torch.int16))
        ops = 2.0 * M * N * K
        res[tag] = dict(M=M, N=N, K=K, bit_identical=same,
                        **{f"{n}_ms": min(t) for n, t in times.items()},
                        **{f"{n}_rounds_ms": [round(v, 4) for v in t] for n, t in times.items()},
                        **{f"{n}_tops": ops / (min(t) * 1e-3) / 1e12 for n, t in times.items()})
        log(f"[bench] 8-wave {tag}: gemm_i8 {min(times['gemm_i8']):.3f} ms, 8-wave {min(times['gemm_i8_8wave']):.3f} "
            f"ms, bit-identical {same}")
        del a, w, ys
    return res


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "one GPU only: the quantized linear path here has no multi-GPU code "
                                   "(its sharding is a design, not an implementation); run with --gpus 1"}))
        sys.exit(2)
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.calibrate_copy:
        n = 1 << 28   # 2^28 fp32 = 1 GiB read and 1 GiB written per launch
        x = torch.ones(n, device="cuda")
        y = torch.empty_like(x)
        for _ in range(3):
            torch.neg(x, out=y)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "torch.neg fp32 elementwise", "bytes_read_per_launch": 4 * n,
                          "bytes_written_per_launch": 4 * n, "launches": 3}))
        return
    from powershard_amd import _native
    _native.lib()
    h, sample = headline(args)
    parity = check_headline_parity(sample)
    log(f"[bench] headline parity ({parity['rows_checked']} sampled rows vs oracle): {parity}")
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(sample, cpu_inputs(sample), args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu['value'] * 1e3:.1f} GOPS on {cpu['cores']} threads "
            f"({cpu['single_thread']['value'] * 1e3:.1f} on one), {cpu['cpu_model']}")
    extra = {}
    if not args.no_extra:
        for name, fn in (("int4_w4a16", extra_int4), ("fp8", extra_fp8), ("w8a16", extra_w8a16),
                         ("wan_ffn_gelu", extra_ffn), ("h3_mlp_silu_gate", extra_h3_mlp),
                         ("shard_m4095", extra_shard),
                         ("wan14b_stack", extra_wan_stack), ("gemm_i8_8wave", extra_8wave)):
            if args.extras and name not in args.extras.split(","):
                continue
            if name == "gemm_i8_8wave" and not args.extras:   # a comparison, run only when named
                continue
            try:
                extra[name] = fn(args)
            except torch.cuda.OutOfMemoryError as e:
                extra[name] = {"error": f"OOM: {e}"}
    traffic = profiled_traffic()
    roof = dict(bound="mfma", achieved=h["gemm_tops"], peak=PEAK_INT8_TOPS, unit="TOPS",
                frac=h["gemm_tops"] / PEAK_INT8_TOPS, traffic=traffic and traffic["bytes"], kernel="gemm_i8",
                kernel_ms=h["gemm_ms"], algorithmic_ops_per_launch=2.0 * h["M"] * h["N"] * h["K"],
                timing="HIP events on the launch stream around back-to-back launches of the GEMM alone",
                traffic_source=traffic and traffic["source"])
    line = {
        "metric": METRIC, "value": round(h["tops"], 2), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(h["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "W8A8 QuantLinear forward with ConvRot (rotate+quantize, int8 MFMA GEMM, "
                               "dequant+bias epilogue), Wan-14B FFN up 5120->13824, M=32760 tokens",
                   "M": h["M"], "K": h["K"], "N": h["N"], "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "kernels": {"gemm_i8_ms": h["gemm_ms"], "quantize_rows_i8_ms": h["quant_ms"],
                    "quantize_rows_i8_gbs": h["quant_gbs"]},
        "parity": parity,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
