"""Benchmark of pico's MI355X backend (one JSON line on stdout).

Workload: fp32 GEMM at M=N=K=4096, entries U[-1,1).
One step = the three products of one matmul's forward and backward
(C = A.B, dA = dC.B^T, dB = A^T.dC), i.e. 3 x 2n^3 FLOP, inputs resident in HBM.
`value` is the achieved TFLOP/s over the timed steps.

Also reported, outside the timed region:
  roofline      the GEMM kernel's FLOP per launch / its mean launch time
                (HIP events on the launch stream) against 157.3 TFLOP/s; its
                HBM bytes per launch come from the committed rocprofv3 PMC
                summary (profiles/traffic.json)
  train         configs 4 and 5: one AdamW training step of the transformer
                built from pico ops (pico_amd/host/gpt.c) per step, tokens/s
  sweep         TFLOP/s for n in {512..8192} and each layout
  row_kernels   RMSNorm / SwiGLU / softmax-CE at the config-3 shapes: GB/s of
                algorithmic traffic against 8 TB/s (buffer sets rotated past
                the 256 MB last-level cache)
  cpu_baseline  pico's own AVX+FMA matmul (threaded, 8 workers) on the host,
                compiled from the reference's sources when present, else this
                repo's restatement of it
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_FP32_PEAK = 157.3e12
MFMA_BF16_PEAK = 2.5e15  # dense bf16 matrix peak (no sparsity)
MFMA_FP8_PEAK = 5.0e15  # dense fp8 matrix peak (no sparsity)
HBM_PEAK = 8.0e12


def _measured_traffic(key):
    """HBM bytes per launch of one kernel, from the committed rocprofv3 PMC
    summary (profiles/traffic.json); None when it has no figure for it"""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)["bytes_per_launch"].get(key)
    except (OSError, ValueError, KeyError):
        return None


def _events_time(fn, reps, warmup):
    """mean ms per call of fn(): `reps` back-to-back launches between two HIP
    events on the launch stream (torch's current stream, which the pk_*
    bindings launch on), so per-launch host gaps are not counted"""
    import torch

    for _ in range(warmup):
        fn()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    ms = s.elapsed_time(e) / reps
    return ms, ms


def _graph_time(fn, reps, warmup):
    """mean ms per call of fn() with the calls captured once into a graph
    (torch.cuda.CUDAGraph over the launch stream) and replayed: back-to-back
    kernels with no host work between them, so a product of a few
    microseconds is not timed as the Python call that launches it"""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(3):
        g.replay()
    e.record()
    e.synchronize()
    del g
    return s.elapsed_time(e) / (3 * reps)


def gemm_section(args, torch, K):
    n = args.n
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(20261201)
    A = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
    B = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
    dC = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
    C = torch.empty(n, n, device=dev)
    dA = torch.empty(n, n, device=dev)
    dB = torch.empty(n, n, device=dev)

    def step():
        K.gemm("N", "N", A, B, C)
        K.gemm("N", "T", dC, B, dA)
        K.gemm("T", "N", A, dC, dB)

    # untimed conditioning: ~0.3 s of the same products first, so the timed
    # steps run at the loaded clock whatever W is (the first launches after an
    # idle spell run slower while the clock ramps up)
    t_end = time.perf_counter() + 0.3
    while time.perf_counter() < t_end:
        step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # timed region: exactly K steps, synchronised on both sides
    t0 = time.perf_counter()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    for i in range(args.steps):
        ev[i][0].record()
        K.gemm("N", "N", A, B, C)
        ev[i][1].record()
        K.gemm("N", "T", dC, B, dA)
        K.gemm("T", "N", A, dC, dB)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    nn_ms = sum(s.elapsed_time(e) for s, e in ev) / len(ev)
    flop_step = 3 * 2.0 * n ** 3
    return {
        "wall_s": wall,
        "value": flop_step * args.steps / wall / 1e12,
        "ms_per_step": wall * 1e3 / args.steps,
        "nn_kernel_ms": nn_ms,
        "flop_per_launch": 2.0 * n ** 3,
    }


def sweep_section(torch, K, sizes, gemm=None):
    gemm = gemm or K.gemm
    dev = torch.device("cuda:0")
    out = {}
    for n in sizes:
        gen = torch.Generator(device=dev).manual_seed(n)
        A = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
        B = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
        C = torch.empty(n, n, device=dev)
        reps = 50 if n <= 1024 else 20 if n <= 2048 else 8 if n <= 4096 else 4
        # untimed conditioning at each size, as for the headline: the clock
        # settles to the load of the new size before its first timed layout
        # (without it the first layout after a smaller size measured 5-6 %
        # slow at 4096^3)
        t_end = time.perf_counter() + 0.1
        while time.perf_counter() < t_end:
            gemm("N", "N", A, B, C)
            torch.cuda.synchronize()
        row = {}
        for ta, tb in (("N", "N"), ("N", "T"), ("T", "N")):
            # replayed from a captured graph: at n <= 1024 a product takes a few
            # microseconds, less than the Python call that launches it
            mean_ms = _graph_time(lambda: gemm(ta, tb, A, B, C), reps, 2)
            row[ta + tb] = round(2.0 * n ** 3 / (mean_ms * 1e-3) / 1e12, 2)
        out[str(n)] = row
        del A, B, C
    return out


def mx8_section(torch, K, sizes):
    """MX8 products (pk_gemm_mx8_f32) with both operands already cast and
    resident, replayed from a graph, and the one-pass casts
    (pk_mx8_quantize_f32) of a row-major and a transposed fp32 operand:
    TFLOP/s against the 5.0 PFLOP/s dense fp8 peak, cast rates in GB/s of
    HBM traffic (4 bytes read + 1 written per value, plus the scales)"""
    dev = torch.device("cuda:0")
    out = {}
    for n in sizes:
        gen = torch.Generator(device=dev).manual_seed(n)
        A = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
        B = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
        C = torch.empty(n, n, device=dev)
        A8, B8 = K.mx8_quantize(A, False), K.mx8_quantize(B, True)
        reps = 20 if n <= 2048 else 8 if n <= 4096 else 4
        t_end = time.perf_counter() + 0.1
        while time.perf_counter() < t_end:
            K.gemm_mx8(n, n, n, A8, B8, C)
            torch.cuda.synchronize()
        ms = _graph_time(lambda: K.gemm_mx8(n, n, n, A8, B8, C), reps, 2)
        qms = _graph_time(lambda: K.mx8_quantize(A, False, out=A8), reps, 2)
        qtms = _graph_time(lambda: K.mx8_quantize(B, True, out=B8), reps, 2)
        tflops = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
        tm, tn, splits = K.mx8_plan(n, n, n)
        out[str(n)] = {"tflops": round(tflops, 1), "frac_of_fp8_peak": round(tflops * 1e12 / MFMA_FP8_PEAK, 4),
                       "us": round(ms * 1e3, 1), "tile": f"{tm}x{tn}", "splits": splits,
                       "cast_us": round(qms * 1e3, 1),
                       "cast_gbs": round(n * n * 5.03 / (qms * 1e-3) / 1e9, 1),
                       "cast_transposed_us": round(qtms * 1e3, 1),
                       "cast_transposed_gbs": round(n * n * 5.03 / (qtms * 1e-3) / 1e9, 1)}
        del A, B, C, A8, B8
    return out


def bf16q_section(torch, K, sizes):
    """bf16 products over bf16 operands held in HBM (pk_gemm_bf16q_f32: the
    narrow-operand kernel with two 32x32x16 bf16 MFMAs per 64-byte slice),
    both operands cast once and resident, replayed from a graph, and the
    one-pass casts (pk_bf16q_quantize_f32): TFLOP/s against the 2.5 PFLOP/s
    dense bf16 peak, cast rates in GB/s (4 bytes read + 2 written per value)"""
    dev = torch.device("cuda:0")
    out = {}
    for n in sizes:
        gen = torch.Generator(device=dev).manual_seed(n)
        A = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
        B = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
        C = torch.empty(n, n, device=dev)
        A16, B16 = K.bf16q_quantize(A, False), K.bf16q_quantize(B, True)
        reps = 20 if n <= 2048 else 8 if n <= 4096 else 4
        t_end = time.perf_counter() + 0.1
        while time.perf_counter() < t_end:
            K.gemm_bf16q(n, n, n, A16, B16, C)
            torch.cuda.synchronize()
        ms = _graph_time(lambda: K.gemm_bf16q(n, n, n, A16, B16, C), reps, 2)
        qms = _graph_time(lambda: K.bf16q_quantize(A, False, out=A16), reps, 2)
        qtms = _graph_time(lambda: K.bf16q_quantize(B, True, out=B16), reps, 2)
        tflops = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
        out[str(n)] = {"tflops": round(tflops, 1), "frac_of_bf16_peak": round(tflops * 1e12 / MFMA_BF16_PEAK, 4),
                       "us": round(ms * 1e3, 1),
                       "cast_gbs": round(n * n * 6 / (qms * 1e-3) / 1e9, 1),
                       "cast_transposed_gbs": round(n * n * 6 / (qtms * 1e-3) / 1e9, 1)}
        del A, B, C, A16, B16
    return out


def bf16x3q_section(torch, K, sizes):
    """fp32 products from three bf16 ones over split-bf16 operands held in HBM
    (pk_gemm_bf16x3q_f32: hi and lo bf16 parts of every value, cast once and
    resident, the narrow-operand kernel with ahi.bhi + ahi.blo + alo.bhi per 16
    values of K), replayed from a graph, and the one-pass casts
    (pk_bf16x3q_quantize_f32): TFLOP/s counted as fp32 products (2n^3), cast
    rates in GB/s (4 bytes read + 4 written per value)"""
    dev = torch.device("cuda:0")
    out = {}
    for n in sizes:
        gen = torch.Generator(device=dev).manual_seed(n)
        A = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
        B = torch.rand(n, n, device=dev, generator=gen) * 2 - 1
        C = torch.empty(n, n, device=dev)
        A3, B3 = K.bf16x3q_quantize(A, False), K.bf16x3q_quantize(B, True)
        reps = 20 if n <= 2048 else 8 if n <= 4096 else 4
        t_end = time.perf_counter() + 0.1
        while time.perf_counter() < t_end:
            K.gemm_bf16x3q(n, n, n, A3, B3, C)
            torch.cuda.synchronize()
        ms = _graph_time(lambda: K.gemm_bf16x3q(n, n, n, A3, B3, C), reps, 2)
        qms = _graph_time(lambda: K.bf16x3q_quantize(A, False, out=A3), reps, 2)
        qtms = _graph_time(lambda: K.bf16x3q_quantize(B, True, out=B3), reps, 2)
        tflops = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
        out[str(n)] = {"tflops": round(tflops, 1), "x_fp32_peak": round(tflops * 1e12 / MFMA_FP32_PEAK, 3),
                       "us": round(ms * 1e3, 1),
                       "cast_gbs": round(n * n * 8 / (qms * 1e-3) / 1e9, 1),
                       "cast_transposed_gbs": round(n * n * 8 / (qtms * 1e-3) / 1e9, 1)}
        del A, B, C, A3, B3
    return out


def attn_section(torch, K):
    """the fused causal attention at config 5's shapes (B 8, H 12, T 1024, hd 64),
    fp32, bf16 and fp8 products (fp8 times include the amax passes over q, k,
    v and dout), randn inputs; TFLOP/s by the causal count (4*hd FLOP per
    visible (query, key) pair forward, 10*hd backward)"""
    dev = torch.device("cuda:0")
    B, H, T, hd = 8, 12, 1024, 64
    D = H * hd
    gen = torch.Generator(device=dev).manual_seed(1)
    q, k, v, do = (torch.randn(B * T, D, device=dev, generator=gen) for _ in range(4))
    o, lse = torch.empty_like(q), torch.empty(B * H * T, device=dev)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    pairs = B * H * T * (T + 1) / 2
    out = {"config": {"batch": B, "heads": H, "seq_len": T, "head_dim": hd}}
    # untimed conditioning, as for the GEMM headline: ~0.2 s of the same
    # launches, so the timed ones run at the loaded clock (the first ~10 ms
    # after an idle spell measured 8-10 % slower)
    t_end = time.perf_counter() + 0.2
    while time.perf_counter() < t_end:
        K.flash_fwd(B, H, q, k, v, o, lse)
        K.flash_bwd(B, H, q, k, v, o, lse, do, dq, dk, dv)
        torch.cuda.synchronize()
    amax = torch.zeros(4, device=dev)
    for name, kw in (("fp32", {}), ("bf16", {"bf16": True}), ("fp8", {"fp8_amax": amax})):
        fwd, _ = _events_time(lambda: K.flash_fwd(B, H, q, k, v, o, lse, **kw), 20, 3)
        bwd, _ = _events_time(lambda: K.flash_bwd(B, H, q, k, v, o, lse, do, dq, dk, dv, **kw),
                              20, 3)
        out[name] = {"fwd_us": round(fwd * 1e3, 1), "bwd_us": round(bwd * 1e3, 1),
                     "fwd_tflops": round(4 * hd * pairs / (fwd * 1e-3) / 1e12, 1),
                     "bwd_tflops": round(10 * hd * pairs / (bwd * 1e-3) / 1e12, 1)}
    # the same kernels on sequences 4x longer: 32 query blocks per head instead
    # of 8, so the causal tail (the last, longest blocks) is a small part of
    # the launch and the rate is the kernels' steady state
    T4 = 4 * T
    q, k, v, do = (torch.randn(B * T4, D, device=dev, generator=gen) for _ in range(4))
    o, lse = torch.empty_like(q), torch.empty(B * H * T4, device=dev)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    pairs4 = B * H * T4 * (T4 + 1) / 2
    fwd, _ = _events_time(lambda: K.flash_fwd(B, H, q, k, v, o, lse), 5, 2)
    bwd, _ = _events_time(lambda: K.flash_bwd(B, H, q, k, v, o, lse, do, dq, dk, dv), 5, 2)
    out["fp32_T4096"] = {"seq_len": T4, "fwd_us": round(fwd * 1e3, 1), "bwd_us": round(bwd * 1e3, 1),
                         "fwd_tflops": round(4 * hd * pairs4 / (fwd * 1e-3) / 1e12, 1),
                         "bwd_tflops": round(10 * hd * pairs4 / (bwd * 1e-3) / 1e12, 1)}
    return out


def rows_section(torch, K):
    """config-3 row kernels; 4 rotating buffer sets (> 256 MB MALL)"""
    dev = torch.device("cuda:0")
    torch.manual_seed(3)  # the row kernels' inputs: torch's seeded device generator
    res = {}
    sets = 4

    def bw(name, nbytes, fns, shape=""):
        i = [0]

        def call():
            fns[i[0] % len(fns)]()
            i[0] += 1

        mean_ms, med_ms = _events_time(call, 20, len(fns))
        gbs = nbytes / (mean_ms * 1e-3) / 1e9
        res[name] = {"us": round(mean_ms * 1e3, 1), "GB/s": round(gbs, 1),
                     "traffic_bytes": _measured_traffic(f"{name} {shape}"),
                     "frac": round(gbs * 1e9 / HBM_PEAK, 3)}

    # context: what a plain device copy (torch's kernel) reaches on this box
    src = [torch.empty(1 << 28, device=dev) for _ in range(sets)]
    dst = [torch.empty(1 << 28, device=dev) for _ in range(sets)]
    bw("copy_1GiB_context", 2 * (1 << 30), [lambda j=j: dst[j].copy_(src[j]) for j in range(sets)])
    del src, dst
    # RMSNorm 8192 x 4096
    R, Cc = 8192, 4096
    xs = [torch.randn(R, Cc, device=dev) for _ in range(sets)]
    ys = [torch.empty(R, Cc, device=dev) for _ in range(sets)]
    g = 1 + 0.02 * torch.randn(Cc, device=dev)
    rs = [torch.empty(R, device=dev) for _ in range(sets)]
    bw("rmsnorm_fwd", 2 * R * Cc * 4,
       [lambda j=j: K.rmsnorm_fwd(xs[j], g, ys[j], rs[j], 1e-6) for j in range(sets)],
       f"{R}x{Cc}")
    dgs = torch.empty(Cc, device=dev)
    ws = torch.empty(K.rmsnorm_bwd_workspace(R, Cc) // 4, device=dev)
    bw("rmsnorm_bwd", 3 * R * Cc * 4,
       [lambda j=j: K.rmsnorm_bwd(xs[j], g, rs[j], ys[(j + 1) % sets], ys[(j + 2) % sets], dgs, ws)
        for j in range(sets)], f"{R}x{Cc}")
    # the part a training step runs on its critical path: dx plus dg's partial
    # sums left in the workspace (their column sum runs on the side stream)
    bw("rmsnorm_bwd_dx_and_partials", 3 * R * Cc * 4,
       [lambda j=j: K.rmsnorm_bwd(xs[j], g, rs[j], ys[(j + 1) % sets], ys[(j + 2) % sets], None,
                                  ws, keep_partials=True)
        for j in range(sets)], f"{R}x{Cc}")
    del xs, ys, rs
    # SwiGLU 8192 x 11008
    R, F = 8192, 11008
    a = [torch.randn(R, F, device=dev) for _ in range(sets)]
    u = [torch.randn(R, F, device=dev) for _ in range(sets)]
    h = [torch.empty(R, F, device=dev) for _ in range(sets)]
    bw("swiglu_fwd", 3 * R * F * 4,
       [lambda j=j: K.swiglu_fwd(a[j], u[j], h[j]) for j in range(sets)], f"{R}x{F}")
    da = [torch.empty(R, F, device=dev) for _ in range(2)]
    bw("swiglu_bwd", 5 * R * F * 4,
       [lambda j=j: K.swiglu_bwd(a[j], u[j], h[j], da[0], da[1]) for j in range(sets)],
       f"{R}x{F}")
    del a, u, h, da
    # softmax-CE 8192 x 32000, fused forward + backward
    R, V = 8192, 32000
    zs = [torch.randn(R, V, device=dev) * 2 for _ in range(2)]
    lab = torch.randint(0, V, (R,), device=dev, dtype=torch.int32)
    loss = torch.empty(R, device=dev)
    dz = [torch.empty(R, V, device=dev) for _ in range(2)]
    bw("xent_fwd_bwd", 2 * R * V * 4,
       [lambda j=j: K.xent_fwd_bwd(zs[j], lab, loss, dz[j], scale=1.0 / R) for j in range(2)],
       f"{R}x{V}")
    return res


TRAIN_CONFIGS = {
    "config4": dict(vocab=8192, d_model=512, n_layers=1, n_heads=8, d_ff=1376, batch=16,
                    seq_len=256),
    "config5": dict(vocab=32000, d_model=768, n_layers=12, n_heads=12, d_ff=2048, batch=8,
                    seq_len=1024),
}
ADAMW = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)


def train_flop_per_step(cfg, causal=True):
    """6 x GEMM params x tokens, plus the attention products (QK^T and PV
    forward, 2x that backward).  causal=True counts the (query, key) pairs the
    kernels compute, T(T+1)/2 per head; causal=False the full T x T that dense
    attention would"""
    d, F, V, L = cfg["d_model"], cfg["d_ff"], cfg["vocab"], cfg["n_layers"]
    T = cfg["seq_len"]
    tok = cfg["batch"] * T
    gemm_params = L * (4 * d * d + 3 * d * F) + d * V
    pairs = T * (T + 1) / 2 if causal else T * T
    attn = L * 3 * 2 * 2 * cfg["batch"] * pairs * d
    return 6.0 * gemm_params * tok + attn


def xorshift_ids(seed, n, vocab):
    """n int32 ids xorshift32() % vocab from `seed`: pico's generator
    (src/tensor.c:249-266, shifts 13/17/5), the synthetic-input recipe for
    labels and token ids"""
    import numpy as np

    s = seed & 0xFFFFFFFF
    out = np.empty(n, np.int32)
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = s % vocab
    return out


def _loss_recorder(P, n):
    """a device buffer of n floats and a function that copies a loss tensor's
    value into slot i on the library's stream (no host synchronisation)"""
    import ctypes

    import torch

    from pico_amd import _lib

    buf = torch.zeros(n, device="cuda:0")
    hip = _lib.hip_lib()
    P.lib.pico_gpu_stream.restype = ctypes.c_void_p

    def record(loss, i):
        st = P.lib.pico_gpu_stream()
        _lib.check("pk_axpy_f32", hip.pk_axpy_f32(1, 1.0, None, loss.contents.data,
                                                   buf.data_ptr() + 4 * i, 0, st))

    return buf, record


def _gpt_step_launches(lib, model, opt, tok, tgt, work):
    loss = lib.pico_gpt_loss(model, tok, tgt)
    if not loss:
        raise RuntimeError("pico_gpt_loss failed")
    lib.pico_optim_adamw_zero_grad(opt)
    lib.pico_backward(work, loss)
    lib.pico_optim_adamw_step(opt)
    return loss


def _graph_replay_ms(P, launch_step, steps):
    """ms per step of a captured step replayed `steps` times (pico_graph_*);
    the step has already run eagerly, so its memory exists"""
    lib = P.lib
    lib.arena_reset(lib.arena_ctx_current())
    if lib.pico_graph_begin() != 0:
        raise RuntimeError(lib.pico_gpu_last_error().decode())
    launch_step()
    graph = lib.pico_graph_end()
    if not graph:
        raise RuntimeError("graph capture failed: " + lib.pico_gpu_last_error().decode())
    for _ in range(2):
        lib.pico_graph_launch(graph)
    P.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        lib.pico_graph_launch(graph)
    P.sync()
    wall = time.perf_counter() - t0
    lib.pico_graph_free(graph)
    lib.arena_reset(lib.arena_ctx_current())
    return wall * 1e3 / steps


SEEDS = {"mlp_x": 20261201, "mlp_labels": 20261202, "mlp_w1": 20261203, "mlp_w2": 20261204,
         "tokens": 20261205, "model_init": 20261201}


def mlp_section(steps, warmup):
    """config 1: pico's 784 -> 128 -> 10 ReLU MLP (examples/02_relu_mlp shapes),
    softmax cross-entropy, SGD lr 0.01, batch 64, inputs resident; eager steps
    and a captured step replayed.  Inputs come from the library's own seeded
    generators: x = pico_randn, W = U(-1/sqrt(fan_in), 1/sqrt(fan_in)) from
    pico_rand, labels xorshift32 % 10, each from a recorded seed."""
    import ctypes

    import numpy as np

    from pico_amd.pico import TP, Pico

    P = Pico()
    lib = P.lib
    x_state = ctypes.c_uint32.in_dll(lib, "x_state")
    data = lib.arena_init(1 << 20)
    lib.arena_ctx_push(data)
    labels = lib.pico_ids_to_device(P.ids(xorshift_ids(SEEDS["mlp_labels"], 64, 10)), 64)
    lib.arena_ctx_pop()
    work = lib.arena_init(1 << 24)
    lib.arena_ctx_push(work)
    fc1 = lib.pico_nn_linear_init(784, 128, True)
    fc2 = lib.pico_nn_linear_init(128, 10, True)
    opt = lib.pico_optim_sgd_init(0.01)
    for fc, (fan, key) in ((fc1, (784, "mlp_w1")), (fc2, (128, "mlp_w2"))):
        w = ctypes.cast(fc + 8, ctypes.POINTER(TP)).contents
        b = ctypes.cast(fc + 16, ctypes.POINTER(TP)).contents
        x_state.value = SEEDS[key]
        u = P.data(P.rand(work, w.contents.shape, w.contents.ndim))
        P.set(w, (2.0 * u.astype(np.float64) - 1.0) * fan ** -0.5)
        lib.pico_optim_sgd_add(opt, w)
        lib.pico_optim_sgd_add(opt, b)
    x_state.value = SEEDS["mlp_x"]
    xs = (ctypes.c_int64 * 2)(64, 784)
    x = P.param([64, 784], P.data(P.randn(work, xs, 2)))
    lib.arena_reset(work)

    def launch_step():
        lib.pico_optim_sgd_zero_grad(opt)
        h = lib.pico_relu(lib.pico_nn_linear_forward(fc1, x))
        loss = lib.pico_softmax_xent(lib.pico_nn_linear_forward(fc2, h), labels)
        lib.pico_backward(work, loss)
        lib.pico_optim_sgd_step(opt)
        return loss

    losses = []
    for _ in range(warmup):
        losses.append(float(P.data(launch_step())[0]))
        lib.arena_reset(work)
    P.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        launch_step()
        lib.arena_reset(work)
    P.sync()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    graph_ms = _graph_replay_ms(P, launch_step, steps)
    err = lib.pico_gpu_last_error().decode()
    lib.arena_ctx_pop()
    lib.pico_optim_sgd_free(opt)
    lib.pico_free(x)
    lib.pico_nn_linear_free(fc1)
    lib.pico_nn_linear_free(fc2)
    lib.arena_destroy(work)
    lib.arena_destroy(data)
    if err:
        raise RuntimeError(err)
    flop = 2 * 64 * (784 * 128 + 128 * 10) * 3
    return {"samples_per_s": round(64 / (ms * 1e-3), 1), "ms_per_step": round(ms, 4),
            "graph_ms_per_step": round(graph_ms, 4),
            "graph_samples_per_s": round(64 / (graph_ms * 1e-3), 1),
            "flop_per_step": flop, "steps": steps, "warmup": warmup,
            "loss_first": round(losses[0], 5), "loss_after_warmup": round(losses[-1], 5),
            "inputs": {"x": f"pico_randn, x_state {SEEDS['mlp_x']}",
                       "w1": f"pico_rand -> U(+-1/sqrt(784)), x_state {SEEDS['mlp_w1']}",
                       "w2": f"pico_rand -> U(+-1/sqrt(128)), x_state {SEEDS['mlp_w2']}",
                       "labels": f"xorshift32 % 10, seed {SEEDS['mlp_labels']}", "biases": 0},
            "config": {"model": "MLP 784-128-10 ReLU", "batch": 64, "optimizer": "SGD lr 0.01"}}


def train_section(name, steps, warmup, precision=0):
    """one AdamW training step of the transformer per step, inputs resident;
    precision 1 runs pico_matmul's products in bf16, 2 as three bf16 products per fp32
    one (pico_set_matmul_precision)"""
    import numpy as np

    from pico_amd.pico import Pico

    cfg = TRAIN_CONFIGS[name]
    P = Pico()
    lib = P.lib
    if lib.pico_set_matmul_precision(precision):
        raise RuntimeError("pico_set_matmul_precision failed")
    model = P.gpt_init(cfg, SEEDS["model_init"])
    n = cfg["batch"] * cfg["seq_len"]
    # synthetic token stream: inputs and next-token targets, xorshift32 % vocab
    seq = xorshift_ids(SEEDS["tokens"], cfg["batch"] * (cfg["seq_len"] + 1), cfg["vocab"])
    seq = seq.reshape(cfg["batch"], cfg["seq_len"] + 1)
    data = lib.arena_init(1 << 20)
    lib.arena_ctx_push(data)
    tok = lib.pico_ids_to_device(P.ids(np.ascontiguousarray(seq[:, :-1])), n)
    tgt = lib.pico_ids_to_device(P.ids(np.ascontiguousarray(seq[:, 1:])), n)
    lib.arena_ctx_pop()
    opt = lib.pico_optim_adamw_init(ADAMW["lr"], ADAMW["beta1"], ADAMW["beta2"], ADAMW["eps"],
                                    ADAMW["weight_decay"])
    for t in P.gpt_params(model):
        lib.pico_optim_adamw_add(opt, t)
    work = lib.arena_init(1 << 30)
    lib.arena_ctx_push(work)
    # the loss of every step, copied on the device into a buffer read once
    # at the end, so recording the curve adds no host synchronisation
    curve, record = _loss_recorder(P, warmup + steps + 1)
    done = [0]

    def step():
        loss = lib.pico_gpt_loss(model, tok, tgt)
        if not loss:
            raise RuntimeError("pico_gpt_loss failed")
        lib.pico_optim_adamw_zero_grad(opt)
        lib.pico_backward(work, loss)
        lib.pico_optim_adamw_step(opt)
        record(loss, done[0])
        done[0] += 1
        lib.arena_reset(work)

    for i in range(warmup):
        step()
    P.sync()
    t0 = time.perf_counter()
    for i in range(steps):
        step()
    P.sync()
    wall = time.perf_counter() - t0
    step()
    P.sync()
    losses = [float(v) for v in curve.cpu().numpy()]
    graph_ms = _graph_replay_ms(P, lambda: _gpt_step_launches(lib, model, opt, tok, tgt, work),
                                steps)
    _, peak_bytes = P.memory()
    err = lib.pico_gpu_last_error().decode()
    lib.arena_ctx_pop()
    lib.arena_destroy(work)
    lib.arena_destroy(data)
    lib.pico_optim_adamw_free(opt)
    lib.pico_gpt_free(model)
    lib.pico_set_matmul_precision(0)
    if err:
        raise RuntimeError(err)
    flop = train_flop_per_step(cfg, causal=True)
    flop_dense = train_flop_per_step(cfg, causal=False)
    ms = wall * 1e3 / steps
    # bf16x3: three bf16 matrix instructions per fp32 product
    peak, peak_name = {1: (MFMA_BF16_PEAK, "bf16 2.5 PFLOP/s"),
                       2: (MFMA_BF16_PEAK / 3, "bf16x3: 2.5 PFLOP/s / 3"),
                       3: (MFMA_FP8_PEAK, "fp8 5.0 PFLOP/s")}.get(
        precision, (MFMA_FP32_PEAK, "fp32 157.3 TFLOP/s"))
    return {"tokens_per_s": round(n * steps / wall, 1), "ms_per_step": round(ms, 3),
            "tflops": round(flop / (ms * 1e-3) / 1e12, 2),
            "mfu": round(flop / (ms * 1e-3) / peak, 4),
            "mfu_count": "causal: attention over the T(T+1)/2 pairs the kernels compute",
            "mfu_dense_count": round(flop_dense / (ms * 1e-3) / peak, 4),
            "flop_per_step": flop, "flop_per_step_dense_attention": flop_dense,
            "mfu_peak": peak_name,
            "graph_ms_per_step": round(graph_ms, 3),
            "graph_tokens_per_s": round(n / (graph_ms * 1e-3), 1),
            "tokens_per_step": n, "steps": steps, "warmup": warmup,
            "loss_first": round(losses[0], 5), "loss_after": round(losses[-1], 5),
            "loss_curve": [round(v, 5) for v in losses],
            "loss_curve_note": f"one batch repeated: {warmup} warmup steps, {steps} timed "
                               "steps, 1 more; each step's loss copied on the device",
            "inputs": {"tokens": f"xorshift32 % vocab, seed {SEEDS['tokens']}",
                       "weights": f"N(0, 0.02) from pico_gpt_init seed {SEEDS['model_init']}"},
            "device_gib_peak": round(peak_bytes / 2 ** 30, 2),
            "optimizer": dict(ADAMW, name="AdamW"), "config": cfg}


def _median_of_3(run):
    """the reference benches' method (bench/bench_matmul_large.c:16-18,42-61):
    one warmup call, then the median of three timed calls, in seconds"""
    run()
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[1]


def cpu_matmul_backward(n):
    """pico's pico_matmul_backward (src/autograd.h:96-130: dA += dC.B^T then
    dB += A^T.dC, scalar, one thread) on n x n operands; 4n^3 FLOP a call"""
    import ctypes

    import numpy as np

    from oracle import oracle as O

    A, B, dC = (O.uniform(n * n, s).reshape(n, n) for s in (1, 2, 3))
    dA, dB = np.zeros((n, n), np.float32), np.zeros((n, n), np.float32)
    if O.ref_available():
        kind, R = "reference", O.ref()

        def run():
            R.picoref_matmul_backward(ctypes.c_int(n), ctypes.c_int(n), ctypes.c_int(n), O.p(A),
                                      O.p(B), O.p(dC), O.p(dA), O.p(dB))
    else:
        kind = "port"

        def run():
            O.matmul_backward(A, B, dC, dA, dB)

    t = _median_of_3(run)
    return {"n": n, "value": round(4.0 * n ** 3 / t / 1e9, 3), "unit": "GFLOP/s", "cores": 1,
            "kind": kind, "s_per_call": round(t, 3),
            "sample": f"pico_matmul_backward at {n}^3 (dA and dB, scalar loops), median of 3 after "
                      "1 warmup"}


def cpu_mlp_steps(steps=100):
    """config 1 on the host: the same 784-128-10 ReLU MLP, softmax-CE and SGD
    lr 0.01 step through the oracle's pico API (pico's CPU path as pico_init
    configures it: the scalar matmul and backward loops, one thread), in the
    pattern of examples/02_relu_mlp/main.c:96-110; the softmax-CE node is the
    oracle's (pico has none).  Median of 3 runs of `steps` steps after 1."""
    import ctypes

    from oracle import oracle as O

    L = O.api()
    keep = L.arena_init(1 << 20)
    L.arena_ctx_push(keep)
    fc1, fc2 = L.pico_nn_linear_init(784, 128, True), L.pico_nn_linear_init(128, 10, True)
    O.set_data(fc1.contents.weights, O.uniform(784 * 128, SEEDS["mlp_w1"], -784 ** -0.5,
                                               784 ** -0.5))
    O.set_data(fc2.contents.weights, O.uniform(128 * 10, SEEDS["mlp_w2"], -128 ** -0.5,
                                               128 ** -0.5))
    opt = L.pico_optim_sgd_init(ctypes.c_float(0.01))
    for fc in (fc1, fc2):
        L.pico_optim_sgd_add(opt, fc.contents.weights)
        L.pico_optim_sgd_add(opt, fc.contents.bias)
    x = O.param([64, 784], O.normal(64 * 784, SEEDS["mlp_x"]))
    labels = O.labels(64, SEEDS["mlp_labels"], 10)
    work = L.arena_init(1 << 24)
    L.arena_ctx_push(work)
    last = [0.0]

    def run():
        for _ in range(steps):
            L.pico_optim_sgd_zero_grad(opt)
            h = L.pico_relu(L.pico_nn_linear_forward(fc1, x))
            loss = L.pico_softmax_xent(L.pico_nn_linear_forward(fc2, h), O.p(labels))
            L.pico_backward(work, loss)
            L.pico_optim_sgd_step(opt)
            last[0] = float(O.data(loss)[0])
            L.arena_reset(work)

    t = _median_of_3(run)
    L.arena_ctx_pop()
    L.arena_destroy(work)
    L.pico_optim_sgd_free(opt)
    L.pico_free(x)
    L.pico_nn_linear_free(fc1)
    L.pico_nn_linear_free(fc2)
    L.arena_ctx_pop()
    L.arena_destroy(keep)
    ms = t * 1e3 / steps
    return {"value": round(64 / (ms * 1e-3), 1), "unit": "samples/s", "ms_per_step": round(ms, 4),
            "cores": 1, "kind": "port", "loss_last": round(last[0], 5),
            "sample": f"{steps} SGD steps of config 1 (batch 64), the oracle's restatement of "
                      "pico's CPU path, median of 3 runs after 1"}


def cpu_baseline(n, bwd_sizes=(1024,)):
    """pico's AVX matmul on the host: warmup 1, median of 3 (bench_matmul_large.c:16-18);
    then pico's scalar matmul backward and a config-1 training step"""
    import ctypes

    import numpy as np

    from oracle import oracle as O

    A = O.uniform(n * n, 1).reshape(n, n)
    B = O.uniform(n * n, 2).reshape(n, n)
    if O.ref_available():
        kind = "reference"
        R = O.ref()

        def run():
            C = np.zeros((n, n), np.float32)
            R.picoref_matmul_avx(ctypes.c_int(n), ctypes.c_int(n), ctypes.c_int(n), O.p(A), O.p(B),
                                 O.p(C))
    else:
        kind = "port"
        O.set_threads(8)

        def run():
            O.matmul_avx(A, B)

    t = _median_of_3(run)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(2.0 * n ** 3 / t / 1e12, 4), "unit": "TFLOP/s", "cores": 8,
            "kind": kind, "host_cpus": os.cpu_count(), "cpu_model": model,
            "sample": f"one fp32 matmul {n}^3 (forward A.B), pico's AVX+FMA kernel on its 8-worker "
                      f"pool, median of 3 after 1 warmup, {t:.2f} s each",
            "matmul_backward": [cpu_matmul_backward(m) for m in bwd_sizes],
            "config1_mlp_step": cpu_mlp_steps()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n", type=int, default=4096)
    ap.add_argument("--sections", default="train,sweep,bf16,fp8,attn,rows,cpu")
    ap.add_argument("--train-steps", type=int, default=50)
    ap.add_argument("--variant-steps", type=int, default=10)
    ap.add_argument("--train-configs", default=",".join(["config1"] + list(TRAIN_CONFIGS)))
    # pico's scalar matmul backward on the host: 1024 takes ~10 s a call, 2048
    # over a minute, so the default run times 1024 only
    ap.add_argument("--cpu-bwd-sizes", default="1024")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU data-parallel path is design-only)", file=sys.stderr)
        sys.exit(2)

    import torch

    from pico_amd import kernels as K

    sections = set(s for s in args.sections.split(",") if s)
    info = K.device_info()
    g = gemm_section(args, torch, K)
    achieved = g["flop_per_launch"] / (g["nn_kernel_ms"] * 1e-3)
    line = {
        "metric": "train tokens/sec (fwd+bwd) + fp32 GEMM TFLOPS, % of MFMA/HBM roofline",
        "value": round(g["value"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic U[-1,1) operands, resident in HBM",
        "config": {"workload": f"fp32 GEMM sweep point M=N=K={args.n}: A.B, dC.B^T, A^T.dC",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 2),
                     "peak": MFMA_FP32_PEAK / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_FP32_PEAK, 4),
                     "traffic": _measured_traffic(f"gemm_f32_kernel<N,N> {args.n}^3"),
                     "traffic_source": "profiles/traffic.json (rocprofv3 FETCH_SIZE x2.00 + "
                                       "WRITE_SIZE x1.00, calibrated on a 256 MiB copy)",
                     "kernel": "gemm_f32_kernel<N,N> (one launch = 2n^3 FLOP)",
                     "kernel_ms": round(g["nn_kernel_ms"], 4)},
        "device": info,
    }
    if "calib" in sections:
        # a plain copy of known size (256 MiB read + 256 MiB written per launch):
        # the yardstick that scales rocprofv3's FETCH_SIZE / WRITE_SIZE to bytes
        src = torch.empty(1 << 26, device="cuda:0").uniform_()
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if "train" in sections:
        line["train"] = {}
        for name in args.train_configs.split(","):
            if name == "config1":
                line["train"][name] = mlp_section(100, 3)
            elif name:
                line["train"][name] = train_section(name, args.train_steps, 3)
    if "sweep" in sections:
        line["sweep"] = sweep_section(torch, K, [512, 1024, 2048, 4096, 8192])
        # the headline kernel again, timed where the sweep times it (after the
        # training sections, on a warm chip) rather than first in the run
        line["roofline"]["achieved_in_sweep_position"] = line["sweep"]["4096"]["NN"]
        line["roofline"]["frac_in_sweep_position"] = round(
            line["sweep"]["4096"]["NN"] * 1e12 / MFMA_FP32_PEAK, 4)
    if "bf16" in sections:
        # outside the fp32 parity contract: bf16 multiplies, fp32 accumulation,
        # fp32 tensors (pk_gemm_bf16_f32 / pico_set_matmul_precision)
        line["bf16"] = {
            "sweep": sweep_section(torch, K, [1024, 2048, 4096, 8192], K.gemm_bf16),
            "bf16q": bf16q_section(torch, K, [2048, 4096, 8192]),
            "train": {name: train_section(name, args.variant_steps, 3, precision=1)
                      for name in args.train_configs.split(",") if name in TRAIN_CONFIGS},
            "peak_tflops": MFMA_BF16_PEAK / 1e12,
            "note": "sweep: bf16 products of fp32 operands (rounded to nearest even on the "
                    "way to LDS), fp32 accumulation; bf16q: bf16 operands cast once and "
                    "resident (pk_gemm_bf16q_f32); train: pico_set_matmul_precision("
                    "PICO_MATMUL_BF16) on the fp32-operand kernels; not the headline, which "
                    "is fp32"}
        # three bf16 products per fp32 one (hi/lo operand split): within ~1e-5 of
        # fp32; TFLOP/s counted as fp32 products (2n^3), not bf16 instructions
        line["bf16x3"] = {
            "sweep": sweep_section(torch, K, [2048, 4096, 8192], K.gemm_bf16x3),
            "bf16x3q": bf16x3q_section(torch, K, [2048, 4096, 8192]),
            "train": {name: train_section(name, args.variant_steps, 3, precision=2)
                      for name in args.train_configs.split(",") if name in TRAIN_CONFIGS},
            "note": "pico_set_matmul_precision(PICO_MATMUL_BF16X3): matmul products as "
                    "ahi.bhi + ahi.blo + alo.bhi in bf16, fp32 accumulation, the fused "
                    "attention's products likewise; bf16x3q: the same products over "
                    "split-bf16 operands cast once and "
                    "resident (pk_gemm_bf16x3q_f32); not the headline, which is fp32"}
    if "fp8" in sections:
        # e4m3 operands (clamped to +-448, nearest even), fp32 accumulation and
        # tensors: far outside the fp32 parity contract, for experiments
        line["fp8"] = {
            "sweep": sweep_section(torch, K, [2048, 4096, 8192], K.gemm_fp8),
            "mx8": mx8_section(torch, K, [2048, 4096, 8192]),
            "train": {name: train_section(name, args.variant_steps, 3, precision=3)
                      for name in args.train_configs.split(",") if name in TRAIN_CONFIGS},
            "note": "sweep: pk_gemm_fp8_f32 (fp32 operands rounded to e4m3 on the way to "
                    "LDS, the 32x32x16 fp8 MFMA); mx8: pk_gemm_mx8_f32 over operands cast once "
                    "to MX8 (e4m3 + a power of two per 32 values) on the 32x32x64 scaled MFMA. "
                    "train: pico_set_matmul_precision(PICO_MATMUL_FP8) -- every product through "
                    "MX8 (weights cast once per optimizer step, activations per product) and "
                    "the fp8 fused attention; not the headline, which is fp32"}
    if "attn" in sections:
        line["attention"] = attn_section(torch, K)
    if "rows" in sections:
        line["row_kernels"] = rows_section(torch, K)
    if "cpu" in sections:
        line["cpu_baseline"] = cpu_baseline(
            args.n, [int(v) for v in args.cpu_bwd_sizes.split(",") if v])
    # the training half of the metric at the top level, and a compact summary
    # as the line's last key (a record that keeps only the end of the line
    # still carries it)
    c5 = line.get("train", {}).get("config5")
    if c5:
        line["train_config"] = "config5 fp32: 12 layers, d 768, batch 8 x seq 1024, AdamW"
        line["train_tokens_per_s"] = c5["tokens_per_s"]
        line["train_ms_per_step"] = c5["ms_per_step"]
        line["train_mfu"] = c5["mfu"]
    summary = {"gemm_4096_tflops": line["value"], "gemm_frac": line["roofline"]["frac"]}
    for name in ("config1", "config4", "config5"):
        t = line.get("train", {}).get(name)
        if t:
            summary[name] = {k: t[k] for k in ("tokens_per_s", "samples_per_s", "ms_per_step",
                                               "graph_ms_per_step", "mfu") if k in t}
    if "sweep" in line:
        summary["sweep_tflops"] = {n: line["sweep"][n]["NN"] for n in line["sweep"]}
    if "attention" in line:
        summary["attention_fp32_us"] = {k: line["attention"]["fp32"][k]
                                        for k in ("fwd_us", "bwd_us")}
    if "row_kernels" in line:
        summary["row_kernels_frac"] = {k: v["frac"] for k, v in line["row_kernels"].items()}
    for prec in ("bf16", "fp8"):
        t5 = line.get(prec, {}).get("train", {}).get("config5")
        if t5:
            summary[f"config5_{prec}_ms_per_step"] = t5["ms_per_step"]
    if "fp8" in line and "mx8" in line["fp8"]:
        summary["mx8_tflops"] = {n: r["tflops"] for n, r in line["fp8"]["mx8"].items()}
    if "bf16" in line and "bf16q" in line["bf16"]:
        summary["bf16q_tflops"] = {n: r["tflops"] for n, r in line["bf16"]["bf16q"].items()}
    if "bf16x3" in line:
        summary["bf16x3q_tflops"] = {n: r["tflops"] for n, r in line["bf16x3"]["bf16x3q"].items()}
    line["summary"] = summary
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
