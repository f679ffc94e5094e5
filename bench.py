"""Benchmark of the decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

Default workload (the headline line): single-token fp16 GEMV at the Llama-3-8B
FFN shapes, W 14336x4096 and 4096x14336, W ~ N(0, 0.02^2), x fp16 ~ N(0, 1),
fp32 accumulation. One step = one GEMV of each shape (an FFN's worth of
weights, 234,991,616 algorithmic bytes). Weights rotate over enough copies
(> 512 MiB) that the 256 MiB Infinity Cache cannot serve them, and all inputs
are resident in HBM before the timed region. The K steps are captured once
into a HIP graph (launches pre-recorded, as the decode engine issues its step)
and replayed; each replay of K steps is bracketed by torch.cuda.synchronize()
and timed with events, and the median of three replays is reported. The same
legs timed as K stream launches from the host are reported beside them
("stream_launched_*").

The line also carries, in "detail", the other legs of the headline metric
measured the same way: int8 block-32 GEMV at the same shapes and decode
attention at L = 32768 (32 Q / 8 KV heads, head_dim 128). "cpu_baseline" is the
C oracle's fp16 GEMV (OpenMP over the host cores) on the 14336x4096 matrix.

Prints ONE JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

PEAK_HBM_GBS = 8000.0
ROTATE_MIN_BYTES = 600 * 2**20
# HBM bytes per launch of the headline kernel from rocprofv3 FETCH_SIZE /
# WRITE_SIZE passes (calibrated against a copy of known size), committed as a
# text summary beside the other profiles.
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gemv_f16_ffn_hbm_traffic.md")


def measured_traffic() -> int | None:
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _events_time(fn, steps: int, warmup: int) -> float:
    """Average ms per call of fn(i) over `steps` calls after `warmup` calls."""
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(warmup + i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def _graph_time(fn, cap, steps: int, warmup: int, reps: int = 3) -> float:
    """Average ms per call of fn(i), i < steps, with the calls captured once
    into a HIP graph on the side stream `cap` (fn must launch on it) and
    replayed: the launches are pre-recorded, as the decode engine issues its
    step, so the events time the kernels and the hardware's gap between them
    rather than the host's launch path. `warmup` eager calls and one replay
    come first; the median of `reps` timed replays of `steps` calls each."""
    import torch

    for i in range(warmup):
        fn(i)
    cap.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        for i in range(steps):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / steps)
    return sorted(times)[len(times) // 2]


def _copies(nbytes: int) -> int:
    return max(3, math.ceil(ROTATE_MIN_BYTES / nbytes))


def _bound(name: str, *args):
    """A closure that calls one C-ABI entry point with pre-resolved arguments.
    The timed loops use these instead of the torch-level operators so that the
    host enqueues faster than the GPU drains (a launch costs ~2 us of Python
    here against kernels of 10+ us), i.e. the events time the kernels."""
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    fn = getattr(_lib.load(), name)

    def run(*_):
        rc = fn(*args)
        if rc:
            raise RuntimeError(f"{name}: {_lib.last_error()}")

    return run


def _stream() -> int:
    import torch

    return torch.cuda.current_stream().cuda_stream


def gemv_f16_leg(steps: int, warmup: int, dev) -> dict:
    import torch

    from gemmagemini4hackathon2026_10_2425_amd import ops

    shapes = [(14336, 4096), (4096, 14336)]
    R = _copies(14336 * 4096 * 2)
    mats = {s: [ops.fill_normal(s, torch.float16, 7, 100 + i, 0.02, dev) for i in range(R)] for s in shapes}
    xs = {s: ops.fill_normal((s[1],), torch.float16, 7, 90, 1.0, dev) for s in shapes}
    ys = {s: torch.empty(s[0], dtype=torch.float32, device=dev) for s in shapes}
    nbytes = {s: s[0] * s[1] * 2 + s[1] * 2 + s[0] * 4 for s in shapes}
    cap = torch.cuda.Stream()

    def bind(st):
        return {s: [_bound("mxd_matvec_f16", W.data_ptr(), xs[s].data_ptr(), 1, ys[s].data_ptr(), s[0], s[1], 0, None,
                           st) for W in mats[s]] for s in shapes}

    calls, gcalls = bind(_stream()), bind(cap.cuda_stream)
    ops.matvec_f16(mats[shapes[0]][0], xs[shapes[0]], ys[shapes[0]])  # argument checks once, through the operator
    per, per_stream = {}, {}
    for s in shapes:
        per[s] = _graph_time(lambda i, s=s: gcalls[s][i % R](), cap, steps, warmup)
        per_stream[s] = _events_time(lambda i, s=s: calls[s][i % R](), steps, warmup)
    ms_step = _graph_time(lambda i: [gcalls[s][i % R]() for s in shapes], cap, steps, warmup)
    ms_step_stream = _events_time(lambda i: [calls[s][i % R]() for s in shapes], steps, warmup)
    step_bytes = sum(nbytes.values())
    return {
        "ms_per_step": ms_step,
        "gbs": step_bytes / ms_step / 1e6,
        "step_bytes": step_bytes,
        "per_shape": {f"{m}x{k}": {"us": per[(m, k)] * 1e3, "bytes": nbytes[(m, k)],
                                   "gbs": nbytes[(m, k)] / per[(m, k)] / 1e6,
                                   "stream_launched_us": per_stream[(m, k)] * 1e3} for (m, k) in shapes},
        "stream_launched_gbs": step_bytes / ms_step_stream / 1e6,
        "copies": R,
    }


def gemv_size_fit_leg(steps: int, warmup: int, dev) -> dict:
    """The fp16 GEMV (fp16 x, K = 4096) at 7168, 14336 and 28672 rows (58.7,
    117.4 and 234.9 MB of weights, rotated copies as in the headline leg) and a
    least-squares fit of time = t0 + bytes / marginal bandwidth. The marginal
    bandwidth is the rate at which the kernel streams once it runs; t0 is the
    fixed cost of one launch (dispatch, the first HBM round trip, the drain),
    which caps the fraction of peak any single call of a given size can reach."""
    import torch

    from gemmagemini4hackathon2026_10_2425_amd import ops

    K = 4096
    pts = []
    for M in (7168, 14336, 28672):
        nb = M * K * 2 + K * 2 + M * 4
        R = _copies(M * K * 2)
        mats = [ops.fill_normal((M, K), torch.float16, 7, 200 + i, 0.02, dev) for i in range(R)]
        x = ops.fill_normal((K,), torch.float16, 7, 90, 1.0, dev)
        y = torch.empty(M, dtype=torch.float32, device=dev)
        cap = torch.cuda.Stream()
        calls = [_bound("mxd_matvec_f16", W.data_ptr(), x.data_ptr(), 1, y.data_ptr(), M, K, 0, None, cap.cuda_stream)
                 for W in mats]
        ms = _graph_time(lambda i: calls[i % R](), cap, steps, warmup)
        pts.append((nb, ms * 1e3))
        del mats
    n = len(pts)
    mb, mt = sum(b for b, _ in pts) / n, sum(t for _, t in pts) / n
    slope = sum((b - mb) * (t - mt) for b, t in pts) / sum((b - mb) ** 2 for b, _ in pts)  # us per byte
    return {
        "points": [{"bytes": b, "us": t, "gbs": b / t / 1e3} for b, t in pts],
        "t0_us": mt - slope * mb,
        "marginal_gbs": 1e-3 / slope,
    }


def launch_floor_leg(steps: int, warmup: int, dev) -> dict:
    """The fixed cost of one kernel on this system, without HBM traffic:
    graph-replayed back-to-back launches of a one-workgroup kernel
    (mxd_f32_to_f16 of 256 values: one load and one store per thread), and of
    the fp16 matvec with a single 4096-wide row (one workgroup, 8 KB of
    weights: the matvec's own start-up, first HBM round trip and drain).
    Per-launch period in the graph, and the same launches stream-ordered."""
    import torch

    from gemmagemini4hackathon2026_10_2425_amd import ops

    cap = torch.cuda.Stream()
    src = torch.zeros(256, dtype=torch.float32, device=dev)
    dst = torch.empty(256, dtype=torch.float16, device=dev)
    W = ops.fill_normal((1, 4096), torch.float16, 7, 400, 0.02, dev)
    x = ops.fill_normal((4096,), torch.float16, 7, 401, 1.0, dev)
    y = torch.empty(1, dtype=torch.float32, device=dev)
    out = {}
    for name, args in (("tiny_kernel", ("mxd_f32_to_f16", src.data_ptr(), dst.data_ptr(), 256)),
                       ("matvec_1x4096", ("mxd_matvec_f16", W.data_ptr(), x.data_ptr(), 1, y.data_ptr(), 1, 4096, 0,
                                          None))):
        g = _bound(*args, cap.cuda_stream)
        e = _bound(*args, _stream())
        out[name] = {"graph_us": _graph_time(g, cap, steps * 10, warmup) * 1e3,
                     "stream_us": _events_time(e, steps * 10, warmup) * 1e3}
    return out


def gemv_q8_leg(steps: int, warmup: int, dev) -> dict:
    import numpy as np
    import torch

    from gemmagemini4hackathon2026_10_2425_amd import ops
    from gemmagemini4hackathon2026_10_2425_amd.quant import quantize_q8b32

    out = {}
    for M, K in [(14336, 4096), (4096, 14336)]:
        W = ops.fill_normal((M, K), torch.float16, 7, 300, 0.02, dev).cpu().numpy()
        q, s = quantize_q8b32(W)
        nb = M * K + M * (K // 32) * 2 + K * 2 + M * 4
        R = _copies(nb)
        qd = [torch.from_numpy(q).to(dev) for _ in range(R)]
        sd = [torch.from_numpy(s).to(dev) for _ in range(R)]
        x = ops.fill_normal((K,), torch.float16, 7, 91, 1.0, dev)
        y = torch.empty(M, dtype=torch.float32, device=dev)
        ops.matvec_q8b32(qd[0], sd[0], x, y)
        cap = torch.cuda.Stream()

        def bind(st):
            return [_bound("mxd_matvec_q8b32", qd[i].data_ptr(), sd[i].data_ptr(), x.data_ptr(), 1, y.data_ptr(), M,
                           K, 0, None, st) for i in range(R)]

        calls, gcalls = bind(_stream()), bind(cap.cuda_stream)
        ms = _graph_time(lambda i: gcalls[i % R](), cap, steps, warmup)
        ms_stream = _events_time(lambda i: calls[i % R](), steps, warmup)
        out[f"{M}x{K}"] = {"us": ms * 1e3, "bytes": nb, "gbs": nb / ms / 1e6, "frac": nb / ms / 1e6 / PEAK_HBM_GBS,
                           "stream_launched_us": ms_stream * 1e3}
        del qd, sd, W, q, s
        np.random.default_rng(0)
    return out


def attention_leg(steps: int, warmup: int, dev, L: int = 32768) -> dict:
    import torch

    from gemmagemini4hackathon2026_10_2425_amd import ops

    nh, nkv, hd = 32, 8, 128
    max_ctx = L
    kv_bytes = 2 * nkv * max_ctx * hd * 2
    R = _copies(kv_bytes)
    ks = [ops.fill_normal((nkv, max_ctx, hd), torch.float16, 8, 10 + i, 1.0, dev) for i in range(R)]
    vs = [ops.fill_normal((nkv, max_ctx, hd), torch.float16, 8, 50 + i, 1.0, dev) for i in range(R)]
    q = ops.fill_normal((nh * hd,), torch.float32, 8, 1, 1.0, dev)
    out = torch.empty(nh * hd, dtype=torch.float32, device=dev)
    ws = ops.attention_workspace(nh, nkv, hd, max_ctx, dev)
    ops.attention(q, ks[0], vs[0], L, nh, out=out, workspace=ws)
    cap = torch.cuda.Stream()

    def bind(st):
        return [_bound("mxd_attention", q.data_ptr(), ks[i].data_ptr(), vs[i].data_ptr(), out.data_ptr(), nh, nkv, hd,
                       max_ctx, L, None, 1.0 / math.sqrt(hd), ws.data_ptr(), ws.numel(), st) for i in range(R)]

    calls, gcalls = bind(_stream()), bind(cap.cuda_stream)
    ms = _graph_time(lambda i: gcalls[i % R](), cap, steps, warmup)
    ms_stream = _events_time(lambda i: calls[i % R](), steps, warmup)
    nb = 4096 * L + nh * hd * 4 * 2
    return {"L": L, "us": ms * 1e3, "bytes": nb, "gbs": nb / ms / 1e6, "frac": nb / ms / 1e6 / PEAK_HBM_GBS,
            "stream_launched_us": ms_stream * 1e3}


def copy_leg(steps: int, warmup: int, dev) -> dict:
    """A plain 1 GiB device-to-device copy (torch's copy kernel): the measured
    copy roof, and the known-size kernel that calibrates HBM byte counters
    (FETCH_SIZE / WRITE_SIZE) for the other kernels."""
    import torch

    n = 2**29
    a = torch.ones(n, dtype=torch.float16, device=dev)
    b = torch.empty_like(a)
    ms = _events_time(lambda i: b.copy_(a), steps, warmup)
    return {"bytes_read": 2 * n, "bytes_written": 2 * n, "us": ms * 1e3, "gbs": 4 * n / ms / 1e6}


def ragged_layer_leg(steps: int, warmup: int, dev, n_seqs: int = 64) -> dict:
    """One Llama-3-8B-shaped layer (hidden 4096, 32 Q / 8 KV heads, head_dim
    128, SwiGLU 14336, int8 block-32 weights) stepping a ragged batch of 64
    sequences with KV lengths uniform in [128, 8192] over a shuffled pool of
    16-key pages. The step (10 launches) is captured once into a graph and
    replayed; every replay appends at the same positions, so the work per
    step is fixed. Bytes per step: the layer's weights once plus every
    sequence's K and V once."""
    import numpy as np
    import torch

    from gemmagemini4hackathon2026_10_2425_amd import _lib, batch, ops

    shape = batch.LLAMA3_8B_LAYER
    lens = np.random.default_rng(20261201).integers(128, 8193, n_seqs) + 1  # + this step's token
    table, n_pages = batch.pack_ragged(lens, seed=5)
    cache = batch.PagedCache(1, shape.n_kv_heads, shape.head_dim, table, n_pages, device=dev)
    st = _stream()
    for pool, tid in ((cache.k, 1), (cache.v, 2)):
        _lib.call("mxd_fill_normal", pool.data_ptr(), _lib.MXD_F16, pool.numel(), 5, tid, 1.0, st)
    layer = batch.RaggedLayerQ8(shape, batch.random_layer_weights(shape, 5), n_seqs, int(lens.max()), dev)
    X = ops.fill_normal((n_seqs, shape.dim), torch.float32, 5, 3, 1.0, dev)
    seq = torch.from_numpy(lens.astype(np.int32)).to(dev)

    def step():
        layer.step(X, cache.k[0], cache.v[0], cache.table, seq)

    step()  # eager once (argument checks)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    ms = _events_time(lambda i: graph.replay(), steps, warmup)
    kv_bytes = int(lens.sum()) * shape.n_kv_heads * shape.head_dim * 2 * 2
    act_bytes = n_seqs * (shape.dim * 4 * 4 + shape.qkv_dim * 4 * 2 + shape.ffn_dim * 6)
    nb = shape.weight_bytes + kv_bytes + act_bytes
    flops = 2 * n_seqs * (shape.weight_bytes - 2 * shape.dim * 4) * 16 // 17
    return {"us": ms * 1e3, "bytes": nb, "weight_bytes": shape.weight_bytes, "kv_bytes": kv_bytes,
            "gbs": nb / ms / 1e6, "frac": nb / ms / 1e6 / PEAK_HBM_GBS, "seqs": n_seqs,
            "kv_tokens": int(lens.sum()), "tok_s": n_seqs / ms * 1e3, "gemm_tflops": flops / ms / 1e9}


def _kv_bytes(shape, n_keys: float) -> float:
    """fp16 K and V bytes one decode step reads at n_keys visible keys: every
    layer's cache (Gemma-4: the layer it reads, the last `window` keys on a
    sliding layer)."""
    from gemmagemini4hackathon2026_10_2425_amd.engine import Gemma4Shape

    if isinstance(shape, Gemma4Shape):
        return sum(2 * 2 * shape.n_kv_heads * y.head_dim * (min(n_keys, shape.window) if y.sliding else n_keys)
                   for y in shape.layers)
    return 2 * 2 * shape.n_layers * shape.n_kv_heads * shape.head_dim * n_keys


def decode_leg(n_new: int = 256, prompt_len: int = 128, reps: int = 3, max_ctx: int | None = None,
               model: str = "gemma2b", window: int = 0) -> dict:
    """Greedy decode of the Gemma-2B, Llama-3.2-1B or Gemma-4-E2B shape, timed like the
    reference's --bench-tg (KL/main.swift:605-618): wall clock over a run of
    pipelined steps that sample on the GPU, one host sync at the end. max_ctx
    defaults to the run's length (384); the serve binary's default is 4096,
    where the attention runs as split + merge launches sized for the whole
    context. With window > 0 the run is the streaming decode the --serve path
    uses (window steps in flight, the host waiting for each token)."""
    import numpy as np

    from gemmagemini4hackathon2026_10_2425_amd.engine import GEMMA4_E2B, GEMMA_2B, LLAMA32_1B, Engine

    shape = {"gemma2b": GEMMA_2B, "llama32_1b": LLAMA32_1B, "gemma4_e2b": GEMMA4_E2B}[model]
    max_ctx = max_ctx or (prompt_len + n_new + 31) // 32 * 32
    with Engine(shape, max_ctx) as e:
        e.init_random(1234)
        prompt = np.random.default_rng(1234).integers(0, shape.vocab, prompt_len).tolist()
        e.set_tokens(prompt)
        e.prefill(prompt_len)
        e.decode(prompt_len, 16)  # warm-up (captures the step graph)
        rates = []
        for _ in range(reps):
            t0 = time.perf_counter()
            if window:
                e.decode_streaming(prompt_len, n_new - 1, lambda t: True, window)
            else:
                e.decode(prompt_len, n_new - 1)
            rates.append((n_new - 1) / (time.perf_counter() - t0))
    rate = float(np.median(rates))
    # bytes per token: every weight once (a tied head is read twice: embed row + head) + the KV read
    per_tok = shape.weight_bytes + _kv_bytes(shape, prompt_len + n_new / 2)
    out = {"tok_s": rate, "ms_per_token": 1e3 / rate, "bytes_per_token": per_tok, "gbs": per_tok * rate / 1e9,
           "frac": per_tok * rate / 1e9 / PEAK_HBM_GBS, "roof_tok_s": PEAK_HBM_GBS * 1e9 / per_tok,
           "prompt": prompt_len, "generated": n_new, "max_ctx": max_ctx}
    if window:
        out["streaming_window"] = window
    return out


def prefill_leg(prompt_len: int = 512, reps: int = 3) -> dict:
    """Gemma-2B-shaped batched prefill of a prompt of random ids (the
    reference's --bench-pp, KL/main.swift:590-603): wall clock over
    Engine.prefill, which ends with a sync. Flops: 2 per weight per prompt row
    in the products (the tied head runs for the last row only)."""
    import numpy as np

    from gemmagemini4hackathon2026_10_2425_amd.engine import GEMMA_2B, Engine

    shape = GEMMA_2B
    max_ctx = (prompt_len + 32 + 31) // 32 * 32
    with Engine(shape, max_ctx) as e:
        e.init_random(1234)
        e.set_tokens(np.random.default_rng(1234).integers(0, shape.vocab, prompt_len).tolist())
        e.prefill(prompt_len)  # warm-up
        rates = []
        for _ in range(reps):
            t0 = time.perf_counter()
            e.prefill(prompt_len)
            rates.append(prompt_len / (time.perf_counter() - t0))
    rate = float(np.median(rates))
    D, F, qkv = shape.dim, shape.ffn_dim, (shape.n_heads + 2 * shape.n_kv_heads) * shape.head_dim
    layer_params = shape.n_layers * (qkv * D + D * shape.n_heads * shape.head_dim + 3 * F * D)
    flops = 2 * layer_params * prompt_len
    return {"prompt": prompt_len, "tok_s": rate, "ms": prompt_len / rate * 1e3,
            "product_tflops": flops / (prompt_len / rate) / 1e12}


def cpu_baseline(seconds: float = 12.0) -> dict:
    """The C oracle's fp16 GEMV (fp64 sums, OpenMP) on the 14336x4096 matrix."""
    import numpy as np

    from oracle import native

    M, K = 14336, 4096
    # Four copies (470 MB) rotate so the host's last-level cache cannot hold them.
    Ws = [native.fill_normal((M, K), np.float16, 7, 100 + i, 0.02) for i in range(4)]
    x = native.fill_normal((K,), np.float16, 7, 90, 1.0).astype(np.float32)
    native.matvec_f16(Ws[0], x)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        native.matvec_f16(Ws[n % 4], x)
        n += 1
    dt = time.perf_counter() - t0
    nb = M * K * 2 + K * 2 + M * 4
    return {
        "value": nb * n / dt / 1e9,
        "unit": "GB/s",
        "cores": native.num_threads(),
        "kind": "port",
        "sample": f"{n} calls of the 14336x4096 fp16 GEMV over 4 rotating copies in {dt:.1f} s (C oracle, "
        f"fp64 sums, {native.num_threads()} OpenMP threads; host has {os.cpu_count()} CPUs)",
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="gemv_f16",
                    choices=["gemv_f16", "gemv_q8", "gemv_size_fit", "launch_floor", "attention", "decode", "decode_4096",
                             "decode_streaming", "decode_llama32_1b", "decode_gemma4_e2b", "prefill", "ragged_layer",
                             "copy"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-detail", action="store_true", help="skip the int8 / attention detail legs")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build has no multi-GPU path)",
              file=sys.stderr)
        return 2

    import torch

    from gemmagemini4hackathon2026_10_2425_amd import _lib

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    detail = {}
    if args.workload != "gemv_f16":
        legs = {"gemv_q8": lambda: gemv_q8_leg(args.steps, args.warmup, dev),
                "launch_floor": lambda: launch_floor_leg(args.steps, args.warmup, dev),
                "gemv_size_fit": lambda: gemv_size_fit_leg(args.steps, args.warmup, dev),
                "attention": lambda: attention_leg(args.steps, args.warmup, dev),
                "decode": decode_leg,
                "decode_4096": lambda: decode_leg(max_ctx=4096),
                "decode_streaming": lambda: decode_leg(max_ctx=4096, window=3),
                "decode_llama32_1b": lambda: decode_leg(model="llama32_1b"),
                "decode_gemma4_e2b": lambda: decode_leg(model="gemma4_e2b"),
                "prefill": prefill_leg,
                "ragged_layer": lambda: ragged_layer_leg(args.steps, args.warmup, dev),
                "copy": lambda: copy_leg(args.steps, args.warmup, dev)}
        print(json.dumps({"workload": args.workload, **legs[args.workload]()}))
        return 0

    log("fp16 GEMV leg")
    g = gemv_f16_leg(args.steps, args.warmup, dev)
    if not args.no_detail:
        log("fp16 GEMV size fit leg")
        detail["gemv_f16_size_fit"] = gemv_size_fit_leg(args.steps, args.warmup, dev)
        detail["launch_floor"] = launch_floor_leg(args.steps, args.warmup, dev)
        torch.cuda.empty_cache()
        log("int8 GEMV leg")
        detail["gemv_q8b32"] = gemv_q8_leg(args.steps, args.warmup, dev)
        log("attention leg")
        detail["attention_L32768"] = attention_leg(args.steps, args.warmup, dev)
        torch.cuda.empty_cache()
        log("decode leg")
        detail["decode_gemma2b"] = decode_leg()
        torch.cuda.empty_cache()
        log("decode leg at the serve default max_ctx 4096")
        detail["decode_gemma2b_maxctx4096"] = decode_leg(max_ctx=4096)
        torch.cuda.empty_cache()
        log("streaming decode leg (window 3, max_ctx 4096)")
        detail["decode_gemma2b_streaming"] = decode_leg(max_ctx=4096, window=3)
        torch.cuda.empty_cache()
        log("Llama-3.2-1B decode leg")
        detail["decode_llama32_1b"] = decode_leg(model="llama32_1b")
        detail["decode_gemma4_e2b"] = decode_leg(model="gemma4_e2b")
        torch.cuda.empty_cache()
        log("ragged batch leg")
        detail["ragged_layer_llama8b_64seq"] = ragged_layer_leg(args.steps, args.warmup, dev)
        torch.cuda.empty_cache()
        log("prefill leg (Gemma-2B, 512-token prompt)")
        detail["prefill_gemma2b_pp512"] = prefill_leg(512)
    detail["gemv_f16"] = g["per_shape"]
    detail["gemv_f16_stream_launched_gbs"] = round(g["stream_launched_gbs"], 1)
    cpu = None
    if not args.no_cpu:
        log("CPU baseline leg")
        cpu = cpu_baseline()
    line = {
        "metric": "GEMV/attention HBM GB/s (% of peak); decode tok/s, Gemma-2B shape, 1 GPU",
        "value": round(g["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (counter-based N(0, 0.02^2) weights, N(0, 1) activations)",
        "config": {
            "workload": "single-token fp16 GEMV, Llama-3-8B FFN shapes 14336x4096 + 4096x14336, fp32 accumulate",
            "weights_rotated_copies": g["copies"],
            "launch": "hip graph of K pre-recorded steps, median of 3 replays",
            "step_bytes": g["step_bytes"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_kernel<fp16 W, fp16 x> (both FFN shapes)",
            "achieved": round(g["gbs"], 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(g["gbs"] / PEAK_HBM_GBS, 4),
            "traffic": measured_traffic(),
            "algorithmic_bytes_per_launch": g["step_bytes"] // 2,
        },
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
