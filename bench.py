"""Benchmark of the FP8 decode-matmul path on one MI355X.

BASELINE.json's metric is quoted at M = 1 and M = 16 (configs[1] "C2" and configs[2] "C3"), so
the default workload (--config decode) measures both in one invocation. A C2 / C3 layer step is
one Qwen3-4B decoder layer's projections - QKV [6144x2560], O [2560x4096], gate_up [19456x2560]
(SwiGLU epilogue), down [2560x9728] - with per-channel FP8 e4m3 weights and per-token dynamic FP8
activation scales, under the reference engine's output contract (engine/engine.py:69, :1005):
QKV split 2, O split 4, down split 4 (fp32 split-K partials), gate_up bf16 SwiGLU. At M = 1 each
projection is one GEMV launch that quantizes its activations itself; at M = 16 the per-token
quantization kernel (quant_rows_tiled) runs before each GEMV. Successive steps use the next of 36
layers of distinct weights (3.6 GB) so the 256 MB MALL cannot serve repeats, as the reference's
tuner cycles layers (engine/engine.py:845-847, :887-891).

Headline: one step = a C2 layer step followed by a C3 layer step (another layer's weights). K
steps are captured into one hipGraph, the graph is replayed R >= 5 times and each replay is timed
with hipEvents between synchronizations: value = algorithmic bytes of the K steps / the median
replay's time (the best replay is reported beside it). Each M is also timed alone the same way
(per_m in the JSON line), with its per-projection table (graph of back-to-back launches cycling
the 36 layers; min and median of 5 replays) and the roofline of its dominant kernel, the gate_up
GEMV, whose HBM traffic comes from the committed rocprofv3 counter summaries
(profiles/traffic_c2.json, traffic_c3.json). Bytes per projection call: N*K (w8) + 4N (w scale)
+ 2MK (bf16 x) + 4M (x scale) + output (2MN bf16, 4SMN partials, 2MI SwiGLU).

Other configs: c2 / c3 / c3m32 (one M alone: 1 / 16 / 32), c4 the lm_head + argmax (--lm
bf16|fp8, --m 1|16), c5 the full decode step (36 layers + lm_head, one graph), layer the fused
FP8 decoder layer (kernels.fused_gemv: O with the residual epilogue, gate_up with the RMSNorm
prologue, down with the residual epilogue, the next QKV with the RMSNorm prologue, chained as
engine/engine.py:953-961 chains them; --m rows), prefill the FP8 prefill GEMM against the library
GEMM (--m rows, default 1024).
"""

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "kernel-rush-qwen_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK = 8.0e12
H, I, NQKV, NQD, V = 2560, 9728, 6144, 4096, 151936
LAYERS = 36
PREFILL_MS = (1024, 4096)  # prompt lengths of the prefill GEMM summary in the default line
METRIC = "FP8 skinny-GEMM HBM GB/s (% of 8 TB/s peak) at Qwen3-4B shapes, M=1 and M=16"
# (name, N rows of W, K, split, mode)
PROJ = [("qkv", NQKV, H, 2, "partial"), ("o", H, NQD, 4, "partial"),
        ("gate_up", 2 * I, H, 1, "swiglu"), ("down", H, I, 4, "partial")]


def fused_layer(torch, dev, layers, xs, M):
    """The fused FP8 decoder layer (engine/engine.py:953-961 order): x = cur + O(attn);
    act = SwiGLU(rmsnorm(x) W_gu); x = x + down(act); qkv = rmsnorm(x) W_qkv (split-2 partials).
    Returns (step, algorithmic bytes per step, [(stage name, fn, bytes)])."""
    from kernels.fused_gemv import FusedLayerBuffers, gemv_fused, gemv_swiglu_fused
    bufs = FusedLayerBuffers(M, H, V, dev)
    g = torch.Generator().manual_seed(3000)
    bufs.res[0].copy_(torch.randn(M, H, generator=g).to(torch.bfloat16))
    ln = [(1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev) for _ in range(2)]
    attn = xs["o"]
    # seed the partials of the first consumers from the starting residual rows
    sq = bufs.res[0].float().pow(2).reshape(M, H // 16, 16).sum(-1)
    bufs.ss[0].copy_(sq)
    bufs.ss[1].copy_(sq)

    def o(i):
        gemv_fused(attn, layers[i % LAYERS]["o"], 4, ep=(bufs.res[0], bufs.res[1], bufs.ss[1], bufs.cnt))

    act = {}

    def gu(i):
        act["a"] = gemv_swiglu_fused(bufs.res[1], layers[i % LAYERS]["gate_up"], norm=(ln[1], bufs.ss[1]))

    gu(0)

    def down(i):
        gemv_fused(act["a"], layers[i % LAYERS]["down"], 4, ep=(bufs.res[1], bufs.res[0], bufs.ss[0], bufs.cnt))

    def qkv(i):
        gemv_fused(bufs.res[0], layers[(i + 1) % LAYERS]["qkv"], 2, norm=(ln[0], bufs.ss[0]))

    def step(i):
        o(i)
        gu(i)
        down(i)
        qkv(i)

    res = 2 * M * H + 2 * M * H + 4 * M * (H // 16)          # residual in / out, sums of squares out
    nrm = 2 * H + 4 * M * (H // 16)                           # RMSNorm weight, sums of squares in
    b_o = H * NQD + 4 * H + 2 * M * NQD + res
    b_gu = 2 * I * H + 8 * I + 2 * M * H + nrm + 2 * M * I
    b_dn = H * I + 4 * H + 2 * M * I + res
    b_qkv = NQKV * H + 4 * NQKV + 2 * M * H + nrm + 4 * 2 * M * NQKV
    stages = [("o+residual", o, b_o), ("gate_up+norm", gu, b_gu), ("down+residual", down, b_dn),
              ("qkv+norm", qkv, b_qkv)]
    return step, b_o + b_gu + b_dn + b_qkv, stages


def static_mlp(torch, fp8, dev, M):
    """The engine's static-scale FP8 decode MLP (engine/engine.py:977-981, both sites FP8):
    delta = linear_fp8(silu_mul(linear_fp8(h, gu8, a_gu)), down8, a_down), with per-tensor
    weights (quantize_weight, as the engine packs gu8 / down8) and SharedScale slots filled from
    the first layer's amax x 2 (the engine's FP8_DECODE_HEADROOM). Returns (the fused step:
    mlp.mlp_fp8_static, two launches; the same on the unfused launches: the SwiGLU GEMV to bf16 act,
    then linear_fp8's cast and down GEMV; algorithmic bytes per step)."""
    from kernels.mlp import mlp_fp8_static
    g = torch.Generator(device=dev)
    layers = []
    for li in range(LAYERS):
        g.manual_seed(5000 + li)
        gu = (torch.randn(2 * I, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        dn = (torch.randn(H, I, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        layers.append((fp8.quantize_weight(gu), fp8.quantize_weight(dn)))
        del gu, dn
    h = torch.randn(M, H, generator=torch.Generator().manual_seed(5100 + M)).to(torch.bfloat16).to(dev)

    def shared(t):
        a = fp8.ActScale(t, headroom=2.0)
        return fp8.SharedScale(a.inv.clone(), a.scale.clone())
    a_gu = shared(h)
    a_dn = shared(fp8.gemv_swiglu_fp8(h, layers[0][0], a=a_gu))

    def fused(i):
        gu8, dn8 = layers[i % LAYERS]
        mlp_fp8_static(h, gu8, dn8, a_gu, a_dn)

    def unfused(i):
        gu8, dn8 = layers[i % LAYERS]
        fp8.linear_fp8(fp8.gemv_swiglu_fp8(h, gu8, a=a_gu), dn8, a_dn)

    nbytes = 2 * I * H + 4 + 2 * M * H + H * I + 4 + 2 * M * H
    return fused, unfused, nbytes


def prefill_times(torch, fp8, M, lin=True):
    """FP8 prefill GEMM at the four Qwen3-4B projections, M rows: krq_gemm_fp8 on e4m3 activations
    against torch._scaled_mm (hipBLASLt) on the same operands, and (lin) the whole linear_fp8
    (ActScale + cast + this GEMM from 128 rows, the library GEMM below). Returns name -> (us ours,
    us library, us linear_fp8 or None, flops), each the minimum over replays of a graph of 20."""
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    out = {}
    for p, (name, N, K, _, _) in enumerate(PROJ):
        g = torch.Generator(device=dev).manual_seed(4000 + p)
        q = fp8.quantize_weight((torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16))
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        a = fp8.ActScale(x)
        x8, xs = fp8._cast(x, a), a.scale.reshape(1)
        t_ours = graph_time(torch, lambda i: fp8.gemm_fp8(x8, q, xs=xs), 20)[0]
        t_lib = graph_time(torch, lambda i: torch._scaled_mm(x8, q[0].t(), scale_a=a.scale, scale_b=q[1],
                                                             out_dtype=torch.bfloat16), 20)[0]
        t_lin = graph_time(torch, lambda i: fp8.linear_fp8(x, q), 20)[0] if lin else None
        fl = 2.0 * M * N * K
        out[name] = (t_ours, t_lib, t_lin, fl)
        log(f"[bench] prefill M={M} {name:<8} krq_gemm_fp8 {t_ours:8.1f} us ({fl / t_ours / 1e6:6.0f} TFLOP/s) | "
            f"hipBLASLt {t_lib:8.1f} us ({fl / t_lib / 1e6:6.0f} TFLOP/s)"
            + (f" | linear_fp8 {t_lin:8.1f} us" if lin else ""))
    return out


def prefill(torch, fp8, dev_rows):
    """--config prefill: prefill_times at M = dev_rows, one JSON line for gate_up."""
    M = dev_rows
    out = prefill_times(torch, fp8, M)
    t_ours, t_lib, t_lin, fl = out["gate_up"]
    tf = fl / t_ours / 1e6
    print(json.dumps({
        "metric": "FP8 prefill GEMM TFLOP/s (gate_up [19456x2560])", "value": round(tf, 1), "unit": "TFLOP/s",
        "n_gpus": 1, "steps": 20, "warmup": 1, "ms_per_step": round(t_ours / 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8_e4m3", "data": "synthetic",
        "config": {"workload": f"prefill GEMM M={M}", "library_tflops": round(fl / t_lib / 1e6, 1),
                   "linear_fp8_us": round(t_lin, 2)},
        "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": 5000.0, "unit": "TFLOP/s",
                     "frac": round(tf / 5000.0, 4), "traffic": None},
        "cpu_baseline": None}), flush=True)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def out_bytes(M, N, split, mode):
    if mode == "partial":
        return 4 * split * M * N
    if mode == "swiglu":
        return 2 * M * (N // 2)
    return 2 * M * N


def chained_mlp(torch, fp8, dev, layers, x):
    """The decode MLP at M = 1 two ways on the same operands: the chained launch
    (PersistentMLP(chained=True), krq_mlp_chain_fp8: gate_up's SwiGLU blocks and down's split-K
    blocks in one launch, the down blocks waiting in the kernel for act) and the two-launch pair
    (gemv_swiglu_fp8, then gemv_fp8 split 4; PersistentMLP's default form). Returns (chained step,
    pair step, algorithmic bytes per step: both weights, scales, x, act written and read, the
    fp32 partials)."""
    from kernels.mlp import PersistentMLP
    pm = PersistentMLP(1, H, I, dev, split=4, chained=True)

    def chain(i):
        Lw = layers[i % LAYERS]
        return pm(x, Lw["gate_up"], Lw["down"])

    def pair(i):
        Lw = layers[i % LAYERS]
        return fp8.gemv_fp8(fp8.gemv_swiglu_fp8(x, Lw["gate_up"]), Lw["down"], 4)
    nbytes = proj_bytes(1, 2 * I, H, 1, "swiglu") + proj_bytes(1, H, I, 4, "partial")
    return chain, pair, nbytes


def proj_bytes(M, N, K, split, mode):
    return N * K + 4 * N + 2 * M * K + 4 * M + out_bytes(M, N, split, mode)


def make_layers(torch, fp8, dev, n_layers):
    """Seeded random-init weights W ~ N(0, 0.02) generated on the device (seed 1000+10l+p),
    quantized per output channel by the HIP quantizer."""
    layers = []
    g = torch.Generator(device=dev)
    for li in range(n_layers):
        L = {}
        for p, (name, N, K, _, _) in enumerate(PROJ):
            g.manual_seed(1000 + 10 * li + p)
            w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            L[name] = fp8.quantize(w)
            del w
        layers.append(L)
    return layers


def make_inputs(torch, dev, M):
    """x ~ N(0, 1) bf16 per projection (seed 2000+p); the down input is SwiGLU of N(0, 1) pairs,
    bf16(bf16(silu(g)) * u) as engine/kernels/ops.py:171-172 rounds it."""
    xs = {}
    for p, (name, N, K, _, _) in enumerate(PROJ):
        g = torch.Generator().manual_seed(2000 + p)
        if name == "down":
            gg = torch.randn(M, K, generator=g).to(torch.bfloat16).float()
            uu = torch.randn(M, K, generator=g).to(torch.bfloat16).float()
            s = (gg / (1.0 + torch.exp(-gg))).to(torch.bfloat16).float()
            xs[name] = (s * uu).to(torch.bfloat16).to(dev)
        else:
            xs[name] = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    return xs


def run_proj(fp8, L_, name, x, split, mode):
    q = L_[name]
    if mode == "swiglu":
        return fp8.gemv_swiglu_fp8(x, q)
    return fp8.gemv_fp8(x, q, split)


def graph_time(torch, fn, reps, iters=5):
    """Capture fn(i) for i in range(reps) into one graph; return (min, median) us per call over
    `iters` replays timed with hipEvents on the capture stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(0)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(reps):
            fn(i)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3 / reps)
    ts.sort()
    del g
    return ts[0], ts[len(ts) // 2]


def kernel_table(torch, fp8, L, layers, xs, M, reps, compare=True):
    """Each kernel of the step alone, back-to-back launches cycling layers (hipEvents around a
    graph replay), each projection the way the step runs it: at M = 1 the GEMV scales its bf16 row
    per token itself (one kernel per projection); at M > 1 quant_rows_tiled runs first and the GEMV
    reads the tiled e4m3 activations. For comparison: at M = 1 the vector-ALU kernel on the same
    operands (name/valu), at M > 1 the GEMV on the same e4m3 rows row-major (name/rowx)."""
    rows = []

    def add(name, N, K, split, mode, fn, xbytes):
        tmin, tmed = graph_time(torch, fn, reps)
        b = N * K + 4 * N + xbytes + 4 * M + out_bytes(M, N, split, mode)
        rows.append(dict(name=name, N=N, K=K, M=M, split=split, mode=mode, us_min=tmin, us_med=tmed,
                         bytes=b, gbs=b / tmed / 1e3, frac=b / (tmed * 1e-6) / HBM_PEAK))

    def bf16_fn(x, name, split, m, algo):
        o = fp8.gemv_fp8_bf16_launch(x, layers[0][name], split, m, None, algo)
        return lambda i: fp8.gemv_fp8_bf16_launch(x, layers[i % len(layers)][name], split, m, None, algo, out=o)

    def tiled_fn(x, name, split, m):
        x8, sc = fp8.quant_rows_tiled(x)
        o = fp8.gemv_fp8_tiled_launch(x8, sc, layers[0][name], M, split, m)
        return lambda i: fp8.gemv_fp8_tiled_launch(x8, sc, layers[i % len(layers)][name], M, split, m, out=o)

    def rowx_fn(x, name, split, m):
        x8, sc = fp8.quant_rows(x)
        sc = sc.reshape(-1)
        o = fp8.gemv_fp8_launch(x8, sc, layers[0][name], split, m)
        return lambda i: fp8.gemv_fp8_launch(x8, sc, layers[i % len(layers)][name], split, m, out=o)

    modes = {"partial": L.OUT_PARTIAL, "swiglu": L.OUT_SWIGLU, "bf16": L.OUT_BF16}
    for name, N, K, split, mode in PROJ:
        x, m = xs[name], modes[mode]
        if M == 1:
            add(name, N, K, split, mode, bf16_fn(x, name, split, m, L.ALGO_AUTO), 2 * M * K)
        else:
            add(name, N, K, split, mode, tiled_fn(x, name, split, m), M * K)
    for name, N, K, split, mode in PROJ if compare else ():
        x, m = xs[name], modes[mode]
        if M == 1:
            add(name + "/valu", N, K, split, mode, bf16_fn(x, name, split, m, L.ALGO_VALU), 2 * M * K)
        else:
            add(name + "/rowx", N, K, split, mode, rowx_fn(x, name, split, m), M * K)
    if M > 1:  # the per-token quantizer launch in front of each GEMV, per activation width
        for name, K in (("quant/qkv,gu", H), ("quant/o", NQD), ("quant/down", I)):
            x = xs["down"] if K == I else xs["o"] if K == NQD else xs["qkv"]
            tq, tqm = graph_time(torch, lambda i: fp8.quant_rows_tiled(x), reps)
            qb = 2 * M * K + 16 * ((M + 15) // 16) * K + 4 * M
            rows.append(dict(name=name, N=0, K=K, M=M, split=1, mode="-", us_min=tq, us_med=tqm,
                             bytes=qb, gbs=qb / tqm / 1e3, frac=qb / (tqm * 1e-6) / HBM_PEAK))
    return rows


def cpu_baseline(torch, Ms, budget_s):
    """The reference's CPU path ("torch dequant+matmul", dequant inside the timed region) on
    this host, over the four projections of one layer at each M in Ms (the headline's halves);
    bounded to about budget_s seconds in all."""
    from oracle import oracle as O
    torch.set_num_threads(os.cpu_count() or 1)
    total_b, total_t, reps_done = 0, 0.0, 0
    g = torch.Generator().manual_seed(0)
    cases = []
    for M in Ms:
        for name, N, K, split, mode in PROJ:
            w8 = (torch.randn(N, K, generator=g) * 200).clamp(-448, 448).to(torch.float8_e4m3fn)
            ws = torch.rand(N, generator=g) * 1e-4
            x8 = (torch.randn(M, K, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
            xs = torch.rand(M, 1, generator=g) * 1e-2
            cases.append((M, name, N, K, w8, ws, x8, xs))
    for c in cases:
        O.torch_dequant_matmul(c[6], c[7], c[4], c[5])   # warm-up
    t_start = time.perf_counter()
    while True:
        for M, name, N, K, w8, ws, x8, xs in cases:
            t0 = time.perf_counter()
            O.torch_dequant_matmul(x8, xs, w8, ws)
            total_t += time.perf_counter() - t0
            total_b += proj_bytes(M, N, K, 1, "bf16")
        reps_done += 1
        if time.perf_counter() - t_start > budget_s or reps_done >= 2000:
            break
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    ms = "+".join(str(m) for m in Ms)
    return {"value": round(total_b / total_t / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{reps_done} passes over the 4 projections of one layer at M={ms} "
                      f"(torch CPU dequant+matmul, bf16 out), {total_t:.1f} s of CPU time; "
                      f"host {model or platform.processor()}, os.cpu_count()={os.cpu_count()}"}


def lm_bytes(M, kind):
    if kind == "bf16":
        return 2 * V * H + 2 * M * H + 8 * M
    return V * H + 4 * V + 2 * M * H + 4 * M + 8 * M


def measured_traffic(cfg, name):
    """(HBM bytes per launch, kernel template) of projection `name` from the committed counter
    summary profiles/traffic_<cfg>.json (FETCH_SIZE + WRITE_SIZE, scaled by a known-size copy),
    or (None, None) when there is none."""
    path = os.path.join(ROOT, "profiles", f"traffic_{cfg}.json")
    try:
        k = json.load(open(path))["projections"][name]
        return int(round(k["read_bytes_median"] + k["write_bytes_median"])), k["kernel"]
    except (OSError, KeyError, ValueError):
        return None, None


def kernel_template(name):
    """A rocprofv3 kernel name without its argument list and namespaces: 'k_gemv_fp8<1, 3, ...>'."""
    name = name.replace("void ", "").replace("(anonymous namespace)::", "")
    return name[:name.index("(")] if "(" in name else name


def summarize_trace(csv_path):
    """Per-kernel durations of a rocprofv3 --kernel-trace CSV (End - Start per dispatch, us).
    'b2b' counts only dispatches whose neighbours in time are the same kernel: the launches of
    the kernel table's graphs (72 back-to-back launches of one kernel), which are what roofline_of
    times with hipEvents. In such a run each dispatch starts when the previous one ends, so its
    traced duration is its share of the run, launch overhead included, like the hipEvents figure.
    'all' counts every dispatch, including those of the mixed step graphs, where the profiler's
    per-dispatch work sits between kernels and stretches the traced spans."""
    import csv
    rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), kernel_template(r["Kernel_Name"]))
                  for r in csv.DictReader(open(csv_path)))
    out = {}
    for i, (s, e, k) in enumerate(rows):
        d = out.setdefault(k, {"all": [], "b2b": []})
        d["all"].append((e - s) / 1000.0)
        if 0 < i < len(rows) - 1 and rows[i - 1][2] == k and rows[i + 1][2] == k:
            d["b2b"].append((e - s) / 1000.0)

    def stats(v):
        return {"n": len(v), "avg_us": round(sum(v) / len(v), 3), "median_us": round(median(sorted(v)), 3)} if v else None
    return {k: {"all": stats(d["all"]), "b2b": stats(d["b2b"])} for k, d in out.items() if k.startswith("k_")}


# The kernel template each step projection runs (tiled weights), per M: the keys of the counter
# summaries profiles/traffic_c2.json / traffic_c3.json that --summarize-pmc writes.
STEP_KERNELS = {
    1: {"qkv": "k_gemv_wide1<1, 1, 10, 5, 4>", "o": "k_gemv_fp8<1, 1, 1, 1, 1, 8, 1, 8>",
        "gate_up": "k_gemv_fp8_swiglu_mixed<1, 1, 1, 5, 5, 1>", "down": "k_gemv_fp8<1, 1, 1, 1, 1, 20, 1, 20>"},
    16: {"qkv": "k_gemv_wide32<1, 10, 48, 1, 1>", "o": "k_gemv_wide32<1, 8, 48, 1, 1>",
         "gate_up": "k_gemv_fp8_swiglu_mixed<1, 3, 1, 5, 0, 1>", "down": "k_gemv_wide32<1, 4, 48, 4, 1>"},
}
PMC_SOURCE = ("rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) --output-format csv -d <out> -o pmc -- python3 bench.py "
              "--no-cpu --no-prefill --no-extra --steps 36 --warmup 2 --reps 36 --replays 1 --calibrate-copy; "
              "then python3 bench.py --summarize-pmc <fetch>/pmc_counter_collection.csv "
              "<write>/pmc_counter_collection.csv <dir>")


def summarize_pmc(fetch_csv, write_csv, out_dir):
    """HBM bytes per dispatch of the step kernels from two rocprofv3 --pmc runs (FETCH_SIZE, then
    WRITE_SIZE, KiB per dispatch), each scaled by what the counter reads for the run's 256 MiB
    device copy (--calibrate-copy: 268,435,456 bytes read and written). Writes traffic_c2.json
    (M = 1) and traffic_c3.json (M = 16) into out_dir; returns their paths."""
    import csv
    from collections import defaultdict

    def load(path, counter):
        vals = defaultdict(list)
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter:
                vals[kernel_template(r["Kernel_Name"])].append(float(r["Counter_Value"]))
        return vals
    F, W = load(fetch_csv, "FETCH_SIZE"), load(write_csv, "WRITE_SIZE")
    copy_f = [max(v) for k, v in F.items() if "copyBuffer" in k]
    copy_w = [max(v) for k, v in W.items() if "copyBuffer" in k]
    if not copy_f or not copy_w:
        raise SystemExit("summarize-pmc: no device copy in the runs (run bench.py with --calibrate-copy)")
    fs, ws = max(copy_f) * 1024 / (256 << 20), max(copy_w) * 1024 / (256 << 20)
    paths = []
    for M, cfg in ((1, "c2"), (16, "c3")):
        out = {"config": cfg, "M": M, "fetch_scale": fs, "write_scale": ws, "source": PMC_SOURCE, "projections": {}}
        for proj, k in STEP_KERNELS[M].items():
            if k not in F or k not in W:
                raise SystemExit(f"summarize-pmc: {k} ({proj}, M={M}) is not in the runs")
            f, w = sorted(F[k]), sorted(W[k])
            out["projections"][proj] = {
                "kernel": k, "read_bytes_median": median(f) * 1024 / fs, "write_bytes_median": median(w) * 1024 / ws,
                "read_bytes_max": f[-1] * 1024 / fs, "dispatches": len(f), "fetch_kib_median": median(f),
                "fetch_kib_max": f[-1], "write_kib_median": median(w)}
        path = os.path.join(out_dir, f"traffic_{cfg}.json")
        with open(path, "w") as fh:
            json.dump(out, fh, indent=1)
        paths.append(path)
    return paths


def traced_us(kernel):
    """Average traced duration (us) of `kernel` over its back-to-back dispatches, from the committed
    kernel-trace summary profiles/gemv_fp8_decode_trace.json (bench.py --summarize-trace), or None."""
    try:
        k = json.load(open(os.path.join(ROOT, "profiles", "gemv_fp8_decode_trace.json")))["kernels"][kernel]
        return k["b2b"]["avg_us"]
    except (OSError, KeyError, ValueError, TypeError):
        return None


def timed_graph(torch, step, steps, warmup, replays):
    """W untimed eager steps, then K steps captured into one graph, replayed once untimed and then
    `replays` times, each replay timed with hipEvents between synchronizations.
    Returns the sorted list of replay times in ms (each for K steps)."""
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(0)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            step(i)
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(replays):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    del g
    return sorted(ts)


def median(ts):
    return ts[len(ts) // 2]


def print_rows(rows, reps):
    log(f"[bench] per-kernel (graph of {reps} back-to-back launches, cycling {LAYERS} layers):")
    log(f"  {'kernel':<14} {'N':>6} {'K':>5} {'M':>3} {'S':>2} {'us(min)':>8} {'us(med)':>8} "
        f"{'bytes':>11} {'GB/s':>7} {'%peak':>6}")
    for r in rows:
        log(f"  {r['name']:<14} {r['N']:>6} {r['K']:>5} {r['M']:>3} {r['split']:>2} {r['us_min']:>8.2f} "
            f"{r['us_med']:>8.2f} {r['bytes']:>11} {r['gbs']:>7.0f} {100 * r['frac']:>5.1f}%")


def roofline_of(rows, M, L, layout, cfg):
    """Roofline of the step's dominant kernel (the GEMV with the largest median time) from the
    kernel table: algorithmic bytes per launch / its median launch time (hipEvents)."""
    dom = max((r for r in rows if r["name"] in ("qkv", "o", "gate_up", "down")), key=lambda r: r["us_med"])
    traffic, kernel = measured_traffic(cfg, dom["name"]) if layout == "tiled" else (None, None)
    a = dom["bytes"] / dom["us_med"] / 1e3
    tr = traced_us(kernel) if kernel else None
    return {"bound": "hbm", "achieved": round(a, 1), "peak": 8000.0, "unit": "GB/s",
            "frac": round(a / 8000.0, 4), "traffic": traffic,
            "kernel": f"gemv_fp8 {dom['name']} [{dom['N']}x{dom['K']}] M={M}" + (f" ({kernel})" if kernel else ""),
            "bytes_per_launch": dom["bytes"], "us_per_launch": round(dom["us_med"], 3),
            "us_per_launch_min": round(dom["us_min"], 3),
            # headline: hipEvents median of this run; beside it the committed kernel trace's average
            # over the same back-to-back launches (profiles/gemv_fp8_decode_trace.json)
            "us_per_launch_trace": tr,
            "frac_trace": round(dom["bytes"] / tr / 1e3 / 8000.0, 4) if tr else None}


def per_m_summary(M, ts, steps, step_bytes, rows, roof):
    t_med, t_min = median(ts), ts[0]
    proj = {r["name"]: {"us_med": round(r["us_med"], 3), "us_min": round(r["us_min"], 3), "bytes": r["bytes"],
                        "gbs": round(r["bytes"] / r["us_med"] / 1e3, 1),
                        "pct_of_hbm_peak": round(100 * r["bytes"] / (r["us_med"] * 1e-6) / HBM_PEAK, 2)}
            for r in rows if "/" not in r["name"]}
    value = step_bytes * steps / (t_med * 1e-3) / 1e9
    return {"M": M, "steps": steps, "replays": len(ts), "ms_per_step": round(t_med / steps, 5),
            "ms_per_step_min": round(t_min / steps, 5), "bytes_per_step": step_bytes,
            "value": round(value, 1), "value_best": round(step_bytes * steps / (t_min * 1e-3) / 1e9, 1),
            "unit": "GB/s", "pct_of_hbm_peak": round(100 * value / 8000.0, 2), "kernels": proj,
            "roofline": roof}


# BASELINE's stated fractions of 8 TB/s per config (C2 / C4 at M = 1: 80%, C3 / C4 at M = 16: 70%)
TARGET = {1: 0.80, 16: 0.70}


def lmhead_summary(torch, fp8, lmhead, G, dev, Ms=(1, 16)):
    """C4: the tied lm_head [V x H] GEMV fused with greedy argmax, BF16 and per-channel FP8
    weights, at each M (graph of 8 launches, min and median of 5 replays)."""
    g = torch.Generator(device=dev).manual_seed(7)
    E = (torch.randn(V, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    q8 = fp8.quantize(E)
    G.pack(E)
    out = {}
    for M in Ms:
        h = torch.randn(M, H, generator=torch.Generator().manual_seed(100 + M)).to(torch.bfloat16).to(dev)
        for kind, w in (("bf16", E), ("fp8", q8)):
            tmin, tmed = graph_time(torch, lambda i: lmhead.lm_head_argmax(h, w), 8)
            b = lm_bytes(M, kind)
            pct = 100 * b / (tmed * 1e-6) / HBM_PEAK
            out[f"{kind}_m{M}"] = {"us_med": round(tmed, 2), "us_min": round(tmin, 2), "bytes": b,
                                   "gbs": round(b / tmed / 1e3, 1), "pct_of_hbm_peak": round(pct, 2),
                                   "target_pct": round(100 * TARGET.get(M, 0.70), 1)}
            log(f"[bench] C4 lm_head {kind} M={M}: {tmed:.2f} us (min {tmin:.2f}), {b / tmed / 1e3:.0f} GB/s, "
                f"{pct:.1f}% of 8 TB/s")
    return out, E


def c5_summary(torch, lmhead, layer_step, layer_bytes, E, dev, Ms=(1, 16)):
    """C5: the full decode-step weight stream, 36 layers x (QKV, O, gate_up, down) FP8 + the BF16
    lm_head with argmax, one hipGraph of 5 steps, min and median of 5 replays, at each M."""
    out = {}
    for M in Ms:
        h = torch.randn(M, H, generator=torch.Generator().manual_seed(100 + M)).to(torch.bfloat16).to(dev)
        layer = layer_step(M)

        def step(i):
            for li in range(LAYERS):
                layer(li)
            lmhead.lm_head_argmax(h, E)
        b = LAYERS * layer_bytes(M) + lm_bytes(M, "bf16")
        ts = timed_graph(torch, step, 5, 1, 5)
        tmed, tmin = median(ts) / 5, ts[0] / 5
        pct = 100 * b / (tmed * 1e-3) / HBM_PEAK
        out[str(M)] = {"ms_per_step": round(tmed, 4), "ms_per_step_min": round(tmin, 4), "bytes_per_step": b,
                       "gbs": round(b / (tmed * 1e-3) / 1e9, 1), "pct_of_hbm_peak": round(pct, 2)}
        log(f"[bench] C5 full step M={M}: {tmed * 1e3:.1f} us (min {tmin * 1e3:.1f}), "
            f"{b / (tmed * 1e-3) / 1e9:.0f} GB/s, {pct:.1f}% of 8 TB/s")
    return out


def m32_summary(torch, fp8, L, layers, layer_step, layer_bytes, dev, reps):
    """C3's second size, M = 32 (16 x 2 tree-verify rows): the step (quant_rows_tiled + GEMV per
    projection, cycling the layers) and each projection's GEMV beside hipBLASLt (torch._scaled_mm)
    on the same shape."""
    M = 32
    xs = make_inputs(torch, dev, M)
    ts = timed_graph(torch, layer_step(M, xs={M: xs}), 72, 2, 5)
    tmed = median(ts) / 72 * 1e3
    rows = kernel_table(torch, fp8, L, layers, xs, M, reps, compare=False)
    lib = prefill_times(torch, fp8, M, lin=False)
    proj = {}
    for r in rows:
        if r["name"] in lib:
            proj[r["name"]] = {"gemv_us": round(r["us_med"], 3), "hipblaslt_us": round(lib[r["name"]][1], 3),
                               "ratio": round(r["us_med"] / lib[r["name"]][1], 3)}
        elif r["name"].startswith("quant"):
            proj[r["name"]] = {"us": round(r["us_med"], 3)}
    b = layer_bytes(M)
    log(f"[bench] M=32 step {tmed:.2f} us, {b / tmed / 1e3:.0f} GB/s; GEMV / hipBLASLt per projection: "
        + ", ".join(f"{k} {v['gemv_us']:.2f}/{v['hipblaslt_us']:.2f}" for k, v in proj.items() if "gemv_us" in v))
    return {"us_per_step": round(tmed, 3), "bytes_per_step": b, "gbs": round(b / tmed / 1e3, 1),
            "pct_of_hbm_peak": round(100 * b / (tmed * 1e-6) / HBM_PEAK, 2), "projections": proj}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--replays", type=int, default=7, help="timed replays of the step graph (>= 5)")
    ap.add_argument("--config", default="decode",
                    choices=["decode", "c2", "c3", "c3m32", "c4", "c5", "layer", "mlp_static", "mlp_chain",
                             "prefill"])
    ap.add_argument("--m", type=int, default=None, help="rows for --config c4 / c5 / layer (default 1) "
                    "and prefill (default 1024)")
    ap.add_argument("--lm", default="bf16", choices=["bf16", "fp8"], help="lm head weights (c4)")
    ap.add_argument("--layout", default="tiled", choices=["tiled", "rowmajor"],
                    help="FP8 weight layout read by the GEMV")
    ap.add_argument("--reps", type=int, default=72, help="launches per graph in the kernel table")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill GEMM summary of the default line")
    ap.add_argument("--no-table", action="store_true", help="skip the per-kernel tables (profiling runs)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the C4 / C5 / M = 32 summaries of the default line (profiling runs)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one 256 MiB device copy (known bytes) to scale HBM counters")
    ap.add_argument("--summarize-pmc", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "DIR"), default=None,
                    help="write DIR/traffic_c2.json and traffic_c3.json from the two counter runs and exit")
    ap.add_argument("--summarize-trace", metavar="CSV", default=None,
                    help="no GPU work: print the per-kernel duration summary of a rocprofv3 kernel-trace CSV "
                    "(this build's kernels; the JSON of profiles/gemv_fp8_decode_trace.json) and exit")
    args = ap.parse_args()
    if args.summarize_pmc:
        for path in summarize_pmc(*args.summarize_pmc):
            print(path)
        return
    if args.summarize_trace:
        print(json.dumps({"source": "rocprofv3 --kernel-trace --stats --output-format csv -d <out> -o kt -- "
                          "python3 bench.py --no-cpu --no-prefill --no-extra; then python3 bench.py "
                          "--summarize-trace <out>/kt_kernel_trace.csv", "kernels": summarize_trace(args.summarize_trace)},
                         indent=1, sort_keys=True))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the path runs on one GPU; sharding across "
              "GPUs is a design note, not an implementation); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.replays < 1:
        sys.exit("bench.py: --replays must be at least 1")

    import torch
    from kernels import _lib as L
    from kernels import fp8, lmhead
    from kernels import gemv as G

    cfg = args.config
    if cfg == "prefill":
        return prefill(torch, fp8, dev_rows=args.m or 1024)
    Ms = {"decode": [1, 16], "c2": [1], "c3": [16], "c3m32": [32]}.get(cfg, [args.m or 1])
    steps = args.steps or {"c4": 20, "c5": 5, "decode": 180}.get(cfg, 360)
    warmup = args.warmup if args.warmup is not None else {"c4": 2, "c5": 1}.get(cfg, 36)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    t0 = time.time()
    layers, xs, E, q8 = None, {}, None, None
    if cfg not in ("c4", "mlp_static"):
        layers = make_layers(torch, fp8, dev, LAYERS)
        if args.layout == "rowmajor":
            layers = [{k: fp8.FP8Weight(q[0], q[1], None) for k, q in Lw.items()} for Lw in layers]
        xs = {M: make_inputs(torch, dev, M) for M in Ms}
    if cfg in ("c4", "c5"):
        g = torch.Generator(device=dev).manual_seed(7)
        E = (torch.randn(V, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        if args.layout == "tiled":
            G.pack(E)
        if cfg == "c4" and args.lm == "fp8":
            q8 = fp8.quantize(E)
            if args.layout == "rowmajor":
                q8 = fp8.FP8Weight(q8[0], q8[1], None)
            E = None
        hg = torch.Generator().manual_seed(100 + Ms[0])
        h = torch.randn(Ms[0], H, generator=hg).to(torch.bfloat16).to(dev)
    torch.cuda.synchronize()
    log(f"[bench] {cfg}: weights ready in {time.time() - t0:.1f} s; M={Ms}")

    def layer_bytes(M):
        return sum(proj_bytes(M, N, K, split, mode) for _, N, K, split, mode in PROJ)

    def layer_step(M, offset=0, xs=xs):
        def step(i):
            Lw = layers[(i + offset) % LAYERS]
            for name, N, K, split, mode in PROJ:
                run_proj(fp8, Lw, name, xs[M][name], split, mode)
        return step

    per_m = {}
    roofline = None
    if cfg in ("decode", "c2", "c3", "c3m32"):
        # the M = 16 half reads layers 18 apart from the M = 1 half of the same step
        parts = [(M, layer_step(M, 18 * j)) for j, M in enumerate(Ms)]

        def step(i):
            for _, fn in parts:
                fn(i)
        step_bytes = sum(layer_bytes(M) for M in Ms)
        ms_list = "+".join(str(M) for M in Ms)
        work = (f"{'C2+C3' if cfg == 'decode' else cfg.upper()}: one Qwen3-4B decoder layer's QKV/O/gate_up/down "
                f"FP8 projections at M={ms_list} (per step, each M on its own layer), per-token dynamic scales, "
                f"per-channel weights, cycling {LAYERS} layers")
    elif cfg == "layer":
        M = Ms[0]
        step, step_bytes, fused_stages = fused_layer(torch, dev, layers, xs[M], M)
        work = (f"fused FP8 decoder layer at M={M}: O + residual, gate_up with RMSNorm, down + residual, "
                f"next QKV with RMSNorm (kernels.fused_gemv), per-token scales, cycling {LAYERS} layers")
    elif cfg == "mlp_static":
        step, unfused_step, step_bytes = static_mlp(torch, fp8, dev, Ms[0])
        work = (f"static-scale FP8 decode MLP at M={Ms[0]} (engine.py:977-981: gate_up with SiLU*up and the "
                f"down input's cast in one launch, then down), per-tensor weights, cycling {LAYERS} layers")
    elif cfg == "mlp_chain":
        step, pair_step, step_bytes = chained_mlp(torch, fp8, dev, layers, xs[1]["gate_up"])
        work = (f"chained FP8 decode MLP at M=1 (gate_up with SwiGLU and down's split-K partials in one launch, "
                f"the down workgroups waiting in the kernel for act), per-token scales, cycling {LAYERS} layers")
    elif cfg == "c4":
        w_lm = E if E is not None else q8
        step = lambda i: lmhead.lm_head_argmax(h, w_lm)
        step_bytes = lm_bytes(Ms[0], args.lm)
        work = (f"C4: tied lm_head [{V}x{H}] {args.lm.upper()} GEMV fused with greedy argmax at M={Ms[0]}")
    else:
        c5_layer = layer_step(Ms[0])

        def step(i):
            for li in range(LAYERS):
                c5_layer(li)
            lmhead.lm_head_argmax(h, E)
        step_bytes = LAYERS * layer_bytes(Ms[0]) + lm_bytes(Ms[0], "bf16")
        work = (f"C5: full decode-step weight stream at M={Ms[0]}: {LAYERS} layers x FP8 QKV/O/gate_up/down "
                f"+ BF16 lm_head with argmax, one hipGraph")

    ts = timed_graph(torch, step, steps, warmup, args.replays)
    t_med, t_min = median(ts), ts[0]
    value = step_bytes * steps / (t_med * 1e-3) / 1e9
    log(f"[bench] {cfg}: {args.replays} replays of {steps} steps: median {t_med / steps * 1e3:.2f} us/step, "
        f"best {t_min / steps * 1e3:.2f} us/step, {value:.0f} GB/s ({100 * value / 8000:.1f}% of 8 TB/s)")

    if cfg in ("decode", "c2", "c3", "c3m32"):
        for M, fn in parts:
            tsm = timed_graph(torch, fn, steps, 0, args.replays) if len(parts) > 1 else ts
            rows = [] if args.no_table else kernel_table(torch, fp8, L, layers, xs[M], M, args.reps)
            if rows:
                print_rows(rows, args.reps)
            tcfg = {1: "c2", 16: "c3", 32: "c3m32"}[M]
            roof = roofline_of(rows, M, L, args.layout, tcfg) if rows else None
            per_m[str(M)] = per_m_summary(M, tsm, steps, layer_bytes(M), rows, roof)
            pm = per_m[str(M)]
            log(f"[bench] M={M} alone: median {pm['ms_per_step'] * 1e3:.2f} us/step (best "
                f"{pm['ms_per_step_min'] * 1e3:.2f}), {pm['value']:.0f} GB/s, {pm['pct_of_hbm_peak']:.1f}% of 8 TB/s")
        roofs = [pm["roofline"] for pm in per_m.values() if pm["roofline"]]
        roofline = max(roofs, key=lambda r: r["us_per_launch"]) if roofs else None

    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log("[bench] calibration copy: 268435456 bytes read, 268435456 bytes written")
        del src, dst

    if cfg == "mlp_static":
        tmin_u, tmed_u = graph_time(torch, unfused_step, args.reps)
        tmin_f, tmed_f = graph_time(torch, step, args.reps)
        log(f"[bench] static-scale MLP M={Ms[0]} (graph of {args.reps}, cycling {LAYERS} layers): fused (SwiGLU GEMV "
            f"casting the down input, down GEMV) {tmed_f:.2f} us (min {tmin_f:.2f}); unfused (SwiGLU GEMV to bf16, "
            f"linear_fp8) {tmed_u:.2f} us (min {tmin_u:.2f})")
        a = step_bytes / tmed_f / 1e3
        roofline = {"bound": "hbm", "achieved": round(a, 1), "peak": 8000.0, "unit": "GB/s",
                    "frac": round(a / 8000.0, 4), "traffic": None, "kernel": f"static-scale FP8 MLP M={Ms[0]}",
                    "bytes_per_launch": step_bytes, "us_per_launch": round(tmed_f, 3),
                    "unfused_us": round(tmed_u, 3)}
    if cfg == "mlp_chain":
        res = {}
        for rnd in range(2):  # alternating, so both forms see the same box state
            for name, fn in (("pair", pair_step), ("chained", step)):
                res.setdefault(name, []).append(graph_time(torch, fn, args.reps))
        (cmin, cmed), (pmin, pmed) = min(res["chained"]), min(res["pair"])
        log(f"[bench] FP8 MLP M=1 (graph of {args.reps}, cycling {LAYERS} layers): chained (one launch) "
            f"{cmed:.2f} us (min {cmin:.2f}); pair (SwiGLU GEMV, down GEMV) {pmed:.2f} us (min {pmin:.2f})")
        a = step_bytes / cmed / 1e3
        roofline = {"bound": "hbm", "achieved": round(a, 1), "peak": 8000.0, "unit": "GB/s",
                    "frac": round(a / 8000.0, 4), "traffic": None, "kernel": "k_mlp_chain_fp8 M=1",
                    "bytes_per_launch": step_bytes, "us_per_launch": round(cmed, 3),
                    "pair_us": round(pmed, 3)}
    if cfg == "layer":
        rows = []
        for name, fn, nbytes in fused_stages:
            tmin, tmed = graph_time(torch, fn, args.reps)
            rows.append({"name": name, "us_min": tmin, "us_med": tmed, "bytes": nbytes})
        log(f"[bench] fused layer stages (graph of {args.reps} back-to-back launches, cycling {LAYERS} layers):")
        for r in rows:
            log(f"  {r['name']:<14} {r['us_min']:8.2f} us (median {r['us_med']:.2f})  {r['bytes']:>10} B  "
                f"{r['bytes'] / r['us_med'] / 1e3:7.0f} GB/s")
        dom = max(rows, key=lambda r: r["us_med"])
        a = dom["bytes"] / dom["us_med"] / 1e3
        roofline = {"bound": "hbm", "achieved": round(a, 1), "peak": 8000.0, "unit": "GB/s",
                    "frac": round(a / 8000.0, 4), "traffic": None, "kernel": f"fused {dom['name']} M={Ms[0]}",
                    "bytes_per_launch": dom["bytes"], "us_per_launch": round(dom["us_med"], 3)}
    elif cfg in ("c4", "c5"):
        w_lm = E if E is not None else q8
        tmin, tmed = graph_time(torch, lambda i: lmhead.lm_head_argmax(h, w_lm), 8 if cfg == "c4" else 4)
        kind = "bf16" if E is not None else "fp8"
        b = lm_bytes(Ms[0], kind)
        a = b / tmed / 1e3
        roofline = {"bound": "hbm", "achieved": round(a, 1), "peak": 8000.0, "unit": "GB/s",
                    "frac": round(a / 8000.0, 4), "traffic": None,
                    "kernel": f"lmhead_argmax {kind} [{V}x{H}] M={Ms[0]}", "bytes_per_launch": b,
                    "us_per_launch": round(tmed, 3), "us_per_launch_min": round(tmin, 3)}
        log(f"[bench] lm_head {kind} M={Ms[0]}: {tmed:.2f} us (min {tmin:.2f}), {a:.0f} GB/s, "
            f"{100 * a / 8000:.1f}% of 8 TB/s")

    cpu = None
    if not args.no_cpu and cfg in ("decode", "c2", "c3", "c3m32"):
        cpu = cpu_baseline(torch, Ms, args.cpu_seconds)
    pre = None
    if cfg == "decode" and not args.no_prefill:
        # the prefill GEMM next to the library's, per decoder layer (the four projections summed)
        pre = {"M": list(PREFILL_MS), "layer_us": [], "hipblaslt_layer_us": [], "ratio": []}
        for pm in PREFILL_MS:
            t = prefill_times(torch, fp8, pm, lin=False)
            ours, lib = sum(v[0] for v in t.values()), sum(v[1] for v in t.values())
            pre["layer_us"].append(round(ours, 1))
            pre["hipblaslt_layer_us"].append(round(lib, 1))
            pre["ratio"].append(round(ours / lib, 3))
        log(f"[bench] prefill GEMM per layer, M={list(PREFILL_MS)}: {pre['layer_us']} us against hipBLASLt "
            f"{pre['hipblaslt_layer_us']} us")
    extra = {}
    if cfg == "decode" and not args.no_extra:
        # BASELINE's other configs beside the headline: C4 (lm_head + argmax), C5 (full step), M = 32
        extra["c4"], E_lm = lmhead_summary(torch, fp8, lmhead, G, dev)
        extra["c5"] = c5_summary(torch, lmhead, layer_step, layer_bytes, E_lm, dev)
        del E_lm
        extra["c3m32"] = m32_summary(torch, fp8, L, layers, layer_step, layer_bytes, dev, args.reps)

    print(json.dumps({
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(t_med / steps, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8_e4m3",
        "data": "synthetic (seeded N(0,0.02) weights generated on device, N(0,1) activations)",
        "config": {"workload": work, "M": Ms if len(Ms) > 1 else Ms[0], "bytes_per_step": step_bytes,
                   "layout": args.layout, "pct_of_hbm_peak": round(100 * value / 8000.0, 2),
                   "replays": args.replays, "ms_per_step_min": round(t_min / steps, 5),
                   "value_best": round(step_bytes * steps / (t_min * 1e-3) / 1e9, 1)},
        "per_m": per_m or None, "prefill": pre, **extra,
        "roofline": roofline, "cpu_baseline": cpu}), flush=True)


if __name__ == "__main__":
    main()
