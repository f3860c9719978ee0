#!/usr/bin/env python3
"""Benchmark of the TinyTransformer inference hot path on one MI355X.

Headline (BASELINE.json ``metric``): greedy decode tokens/s of the small model (d=768, 12 heads,
4 layers, d_ff=2048, bf16) at B=256: 32 synthetic tasks x 8 dihedral /
colour variants, prompts of 300-1800 tokens left-padded into one batch, a 2,048-slot static KV
cache, greedy decode up to 930 tokens (capped by the cache at 2048 - S_pad, as the reference's
``max_total_len`` does).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config small_b256|medium_b128|large_b64]

A *step* is one greedy decode step of the whole B=256 batch (grid state -> embedding -> 4 layers
-> LM head / argmax -> commit), replayed from the captured HIP graph the product path uses.  The
prompt prefill runs once before the timed region (reported separately).  ``value`` =
B * K / (timed seconds).

Also reported on the same JSON line:
* ``roofline``: decode attention (the dominant kernel, HBM-bound).  Its timed-region launches
  are re-issued one by one with HIP events on the launching stream (same layers, same cache
  fills t, same buffers) to get the average launch duration; achieved GB/s = algorithmic bytes
  per launch (K/V slots each row attends, q, output, prompt mask) / that duration.
* ``cpu_baseline``: the fp32 CPU oracle (oracle/reference_path.py) decoding the same B=256 batch
  from the same cache contents for a bounded number of steps on the host cores.
* ``microbench``: BASELINE config 1 -- the fused norm / RoPE / SwiGLU kernels at N=65,536
  tokens, d=768, F=2048, GB/s against the 8 TB/s HBM peak (buffer sets rotated so the 256 MB
  MALL cannot hold the working set): the inference path's forms (fp32 GEMM outputs in, split
  GEMM inputs out) and the ``*_bf16`` forms in config 1's own format (bf16 activations in and
  out); ``frac_of_algorithmic`` divides config 1's algorithmic bytes (bf16 in and out) by the
  kernel time.
* ``prefill_attention``: the prefill attention kernel alone over one layer of the batch's cache
  (its real masks and left padding, packed query rows as the prefill launches it), re-launched
  back to back (median of 5 rounds of 10 launches after 3 warm ones); TFLOP/s of the valid
  causal (query, key) pairs against the 2.5 PFLOP/s dense bf16 MFMA peak, and (``hbm``) the same
  launches' algorithmic bytes (q, the K/V of every valid key once, the hi|lo output) against
  the 8 TB/s HBM peak.

* ``configs``: BASELINE configs 3 (medium, B=128, 4,096-slot cache) and 4 (large, B=64, prompts
  of 5,000-5,726 tokens) measured the same way over 32 graph-replayed steps each: decode
  tokens/s, the decode attention's GB/s, the prefill and one layer's prefill-attention TFLOP/s
  (``--no-side`` skips them).

``roofline.traffic`` is the HBM bytes per launch the rocprofv3 FETCH_SIZE / WRITE_SIZE passes
measured per algorithmic byte (profiles/pmc_traffic_small_b256.md) times this line's own
algorithmic bytes per launch.

``--config medium_b128`` / ``large_b64`` run BASELINE configs 3 and 4 as the headline workload
(their own metric name; no microbench; the CPU baseline only with an explicit ``--cpu-seconds``).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
METRIC = "greedy decode tokens/s at small, B=256; fused-kernel HBM GB/s as % of peak"
WORKLOADS = {
    "small_b256": "BASELINE config 2: small TinyTransformer (d=768, 12 heads, 4 layers, "
                  "d_ff=2048) bf16, random init seed 0, B=256 greedy decode "
                  "(32 tasks x 8 dihedral+colour variants, left-padded)",
    "medium_b128": "BASELINE config 3: medium TinyTransformer (d=1024, 16 heads, 8 layers, "
                   "d_ff=2752) bf16, random init seed 0, B=128 greedy decode (16 tasks x 8 "
                   "variants, 4-5 demo pairs, prompts 1500-3500 tokens, 4096-slot cache)",
    "large_b64": "BASELINE config 4: large TinyTransformer (d=1280, 20 heads, 12 layers, "
                 "d_ff=3392) bf16, random init seed 0, B=64 greedy decode (8 tasks x 8 "
                 "variants, 5 demo pairs, prompts 5000-5726 tokens, 6656-slot cache)",
}


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="small_b256",
                    choices=["small_b256", "medium_b128", "large_b64"],
                    help="BASELINE workload (default: config 2, the headline metric)")
    ap.add_argument("--cpu-seconds", type=float, default=None,
                    help="time bound of the CPU-baseline sample (0 disables it; default 15 s "
                         "for small_b256, off for the larger configs)")
    ap.add_argument("--no-micro", action="store_true", help="skip the config-1 microbench")
    ap.add_argument("--no-side", action="store_true",
                    help="skip the configs 3 and 4 sub-objects of the default (config 2) line")
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel from the host instead of replaying a HIP graph")
    ap.add_argument("--gemm-compare", action="store_true",
                    help="also time the decode projections at this workload's shapes (M = rows): "
                         "K5 (mdl_gemm_split, tiled operands; gate/up with the SwiGLU fused) "
                         "against hipBLASLt on [W | W], each replayed 50x from a HIP graph")
    ap.add_argument("--augment", action="store_true",
                    help="also time predict_with_augmentations on one task of the workload: "
                         "8 dihedral x 8 colour variants in one fused generation against the "
                         "reference's loop over chunks of 16 (same predictions required)")
    return ap.parse_args()


class Timer:
    """HIP events on the current stream."""

    def __init__(self):
        import torch

        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def start(self):
        self.a.record()

    def stop(self):
        self.b.record()

    def ms(self) -> float:
        self.b.synchronize()
        return self.a.elapsed_time(self.b)


def recorded_traffic_ratio(kernel: str, workload: str):
    """HBM bytes per algorithmic byte of ``kernel`` at ``workload``: the rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (calibrated against a device copy) over the same launches' algorithmic
    bytes, recorded in profiles/pmc_traffic_<workload>.md; (None, None) without such a record.
    The bench line's ``traffic`` is this ratio times its own launches' algorithmic bytes."""
    path = os.path.join(ROOT, "profiles", f"pmc_traffic_{workload}.md")
    if not os.path.exists(path):
        return None, None
    key = f"traffic_per_algorithmic_byte {kernel} {workload}:"
    with open(path) as f:
        for line in f:
            if line.startswith(key):
                return float(line[len(key):].strip()), os.path.relpath(path, ROOT)
    return None, None


def decode_attention_bytes(B, H, t, kv_start, S, holes):
    """Algorithmic bytes of one decode-attention launch of the step (mdl_attn_decode; the qkv
    projection's epilogue already wrote q and the token's K/V into slot t) at cache position t:
    every (row, head) reads its bf16 q (64 x 2 B), the K and V rows of the slots it attends
    (kv_start[b]..t, 2 x 128 B each) and writes the split output (2 x 128 B); rows whose prompt
    mask has holes also read their mask bytes."""
    import torch

    ks = kv_start.to(torch.int64)
    n = (t + 1 - ks).clamp(min=0)
    kv = int(n.sum()) * H * 64 * 2 * 2
    q_in = B * H * 64 * 2
    out = B * H * 64 * 2 * 2
    mask = int(((S - ks).clamp(min=0) * holes.to(torch.int64)).sum())
    return kv + q_in + out + mask


def microbench(dev):
    """K1 / K2 / K3 at N = 64 x 1024 tokens, d = 768, 12 heads, F = 2048."""
    import torch

    from mdlarc_scale_amd import kernels as K
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D
    from mdlarc_scale_amd.workload import SPECS, build_prompts, left_pad

    Bm, T, d, H, F = 64, 1024, 768, 12, 2048
    N = Bm * T
    g = torch.Generator(device="cpu").manual_seed(1)
    sets = 3
    # positions from synthetic grids (config 0 generator), tiled to T tokens per row
    prompts = build_prompts(SPECS["tiny_cpu"])
    _, pos_p, _ = left_pad(prompts)
    flat = pos_p.reshape(-1, 3)
    reps = (N + flat.shape[0] - 1) // flat.shape[0]
    pos = flat.repeat(reps, 1)[:N].contiguous().to(dev)
    rope = RotaryEmbedding3D(64, 32, 32, 8)
    tab = rope.device_table(dev)
    geom = (32, 32, 8, rope.px, rope.py, rope.pz)
    res = {}

    def timeit(fn, n_iter=20):
        for i in range(3):
            fn(i % sets)
        t = Timer()
        t.start()
        for i in range(n_iter):
            fn(i % sets)
        t.stop()
        return t.ms() / n_iter

    # K1: embedding gather + example add + RMSNorm -> x fp32, split x*gamma, rstd
    tok = torch.randn(14, d, generator=g).to(dev, torch.bfloat16)
    ex = torch.randn(1280, d, generator=g).to(dev, torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(d, generator=g)).to(dev)
    ids = [torch.randint(0, 14, (N,), generator=g).to(dev) for _ in range(sets)]
    exi = [torch.randint(0, 1280, (Bm,), generator=g).to(dev) for _ in range(sets)]
    xo = [torch.empty(N, d, device=dev) for _ in range(sets)]
    xs = [torch.empty(N, 2 * d, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    rs = [torch.empty(N, device=dev) for _ in range(sets)]
    ms = timeit(lambda i: K.embed_rmsnorm(ids[i], exi[i], tok, ex, T, gamma, 1e-5, xo[i], xs[i],
                                          rs[i]))
    nbytes = N * 8 + N * d * 4 + N * 2 * d * 2 + N * 4
    res["k1_embed_rmsnorm"] = dict(ms=ms, bytes=nbytes, gbs=nbytes / ms / 1e6)
    del xo, xs, rs

    # K2: qkv (fp32 GEMM output) -> rstd scale + split + 3D RoPE + q out + K/V cache write
    qkv = [torch.randn(N, 3 * d, generator=g).to(dev) for _ in range(sets)]
    rstd = [(0.5 + torch.rand(N, generator=g)).to(dev) for _ in range(sets)]
    q = [torch.empty(N, d, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    kc = [torch.empty(Bm, H, T, 64, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    vc = [torch.empty_like(kc[0]) for _ in range(sets)]
    ms = timeit(lambda i: K.qkv_rope_cache(qkv[i], rstd[i], pos, tab, geom, Bm, T, H, 0.125, q[i],
                                           kc[i], vc[i], slot0=0))
    nbytes = N * (3 * d * 4 + 4 + 24 + d * 2 + 2 * d * 2)
    res["k2_qkv_rope_cache"] = dict(ms=ms, bytes=nbytes, gbs=nbytes / ms / 1e6)
    del qkv, rstd, q, kc, vc

    # K3: SwiGLU [N, 2F] fp32 -> split h [N, 2F] bf16
    gu = [torch.randn(N, 2 * F, generator=g).to(dev) for _ in range(sets)]
    rstd = [(0.5 + torch.rand(N, generator=g)).to(dev) for _ in range(sets)]
    bg = (0.1 * torch.randn(F, generator=g)).to(dev)
    bu = (0.1 * torch.randn(F, generator=g)).to(dev)
    h = [torch.empty(N, 2 * F, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    ms = timeit(lambda i: K.swiglu(gu[i], rstd[i], bg, bu, h[i]))
    nbytes = N * (2 * F * 4 + 4 + 2 * F * 2)
    res["k3_swiglu"] = dict(ms=ms, bytes=nbytes, gbs=nbytes / ms / 1e6)
    del gu, h

    # residual add (+ fc_down bias) + next RMSNorm: x += delta + b in place, rstd, split(x*gamma)
    x = [torch.randn(N, d, generator=g).to(dev) for _ in range(sets)]
    delta = [torch.randn(N, d, generator=g).to(dev) for _ in range(sets)]
    bias = (0.1 * torch.randn(d, generator=g)).to(dev)
    xs = [torch.empty(N, 2 * d, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    ms = timeit(lambda i: K.add_rmsnorm(x[i], delta[i], bias, gamma, 1e-5, xs[i], rstd[i]))
    nbytes = N * (d * 4 * 2 + d * 4 + d * 2 * 2 + 4)
    res["add_rmsnorm"] = dict(ms=ms, bytes=nbytes, gbs=nbytes / ms / 1e6)
    del x, delta, xs, rstd

    # the same three kernels in config 1's own format: bf16 activations in and out
    ids = [torch.randint(0, 14, (N,), generator=g).to(dev) for _ in range(sets)]
    xb = [torch.empty(N, d, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    xn = [torch.empty(N, d, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    ms = timeit(lambda i: K.embed_rmsnorm_bf16(ids[i], exi[i], tok, ex, T, gamma, 1e-5, xb[i],
                                               xn[i]))
    nbytes = N * 8 + N * d * 2 * 2
    res["k1_embed_rmsnorm_bf16"] = dict(ms=ms, bytes=nbytes, gbs=nbytes / ms / 1e6)
    del xb, xn
    qkvb = [torch.randn(N, 3 * d, generator=g).to(dev, torch.bfloat16) for _ in range(sets)]
    rstd = [(0.5 + torch.rand(N, generator=g)).to(dev) for _ in range(sets)]
    q = [torch.empty(N, d, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    kc = [torch.empty(Bm, H, T, 64, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    vc = [torch.empty_like(kc[0]) for _ in range(sets)]
    ms = timeit(lambda i: K.qkv_rope_cache_bf16(qkvb[i], rstd[i], pos, tab, geom, Bm, T, H, 0.125,
                                                q[i], kc[i], vc[i], slot0=0))
    nbytes = N * (3 * d * 2 + 4 + 24 + 3 * d * 2)     # positions as the reference's int64
    res["k2_qkv_rope_cache_bf16"] = dict(ms=ms, bytes=nbytes, gbs=nbytes / ms / 1e6)
    del qkvb, rstd, q, kc, vc
    gub = [torch.randn(N, 2 * F, generator=g).to(dev, torch.bfloat16) for _ in range(sets)]
    hb = [torch.empty(N, F, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    ms = timeit(lambda i: K.swiglu_bf16(gub[i], None, bg, bu, hb[i]))
    nbytes = N * (2 * F * 2 + F * 2)
    res["k3_swiglu_bf16"] = dict(ms=ms, bytes=nbytes, gbs=nbytes / ms / 1e6)
    del gub, hb

    # the bytes config 1 defines (bf16 activations in and out): K1 ids + x + normed x;
    # K2 qkv + rstd/positions + q, k, v; K3 gate/up + h.  The kernels above move more: fp32
    # residual / GEMM outputs and hi|lo split GEMM inputs (the parity design's formats)
    algorithmic = {"k1_embed_rmsnorm": N * 8 + N * d * (2 + 2),
                   "k2_qkv_rope_cache": N * (3 * d * 2 + 16 + 3 * d * 2),
                   "k3_swiglu": N * 2 * F * 2 + N * F * 2}
    for name, v in res.items():
        v["frac_of_peak"] = round(v["gbs"] / HBM_PEAK_GBS, 4)
        base = name[:-5] if name.endswith("_bf16") else name
        if base in algorithmic:
            a = algorithmic[base]
            v["algorithmic_bytes"] = a
            v["algorithmic_gbs"] = round(a / v["ms"] / 1e6, 1)
            v["frac_of_algorithmic"] = round(a / v["ms"] / 1e6 / HBM_PEAK_GBS, 4)
        v["ms"] = round(v["ms"], 5)
        v["gbs"] = round(v["gbs"], 1)
    return res


def graph_time_us(fn, reps=50, replays=10):
    """Average duration of ``fn``'s launches replayed from a HIP graph of ``reps`` calls
    (back to back, no host launch gaps)."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):   # capture_begin: no allocator-cache release (capture_greedy)
        g.capture_begin()
        try:
            for _ in range(reps):
                fn()
        finally:
            g.capture_end()
    torch.cuda.current_stream().wait_stream(side)
    g.replay()
    t = Timer()
    t.start()
    for _ in range(replays):
        g.replay()
    t.stop()
    return t.ms() * 1e3 / (reps * replays)


def decode_gemm_compare(cfg, B, dev):
    """The four decode projections of one layer at M = B rows on random bf16 weights: K5 with
    tiled operands (the decode step's form) against hipBLASLt on the [W | W] operand (the form
    before K5), plus the gate / up projection with the SwiGLU fused against K5 + K3."""
    import torch

    from mdlarc_scale_amd import kernels as K
    from mdlarc_scale_amd.engine import gemm_f32

    d, F = cfg.d_model, cfg.d_ff
    g = torch.Generator(device="cpu").manual_seed(3)
    res = {}
    for name, N, k in (("qkv", 3 * d, d), ("out", d, d), ("gate_up", 2 * F, d), ("down", d, F)):
        a = torch.randn(B, 2 * k, generator=g).to(dev, torch.bfloat16)
        w2 = (0.05 * torch.randn(N, 2 * k, generator=g)).to(dev, torch.bfloat16)
        at, wt = K.tile_matrix(a), K.tile_matrix(w2, k)
        out = torch.empty(B, N, device=dev)
        t_blas = graph_time_us(lambda: gemm_f32(a, w2, out))
        t_k5 = graph_time_us(lambda: K.gemm_split(at, wt, out, k, a_tiled=True, w_tiled=True))
        nbytes = N * k * 2 + B * 2 * k * 2 + B * N * 4     # W once, split A, fp32 out
        res[name] = dict(n=N, k=k, tile=K.gemm_split_pick(B, N, k), hipblaslt_us=round(t_blas, 2),
                         k5_us=round(t_k5, 2), bytes=nbytes,
                         k5_gbs=round(nbytes / t_k5 / 1e3, 1))
        if name == "gate_up":
            rstd = (0.5 + torch.rand(B, generator=g)).to(dev)
            bg = (0.1 * torch.randn(F, generator=g)).to(dev)
            bu = (0.1 * torch.randn(F, generator=g)).to(dev)
            h = torch.empty(K.split_numel(B, F, True), device=dev, dtype=torch.bfloat16)
            w_il = K.tile_matrix(K.interleave_gate_up(w2[:F, :k], w2[F:, :k]))
            t_sw = graph_time_us(lambda: K.swiglu(out, rstd, bg, bu, h, tiled=True))
            t_f = graph_time_us(lambda: K.gemm_split_swiglu(at, w_il, rstd, bg, bu, h, B, F, k))
            res[name].update(swiglu_us=round(t_sw, 2), fused_swiglu_us=round(t_f, 2))
    # the decode step's forms: RMSNorm in the qkv / gate-up prologues (x in the fp32 tile
    # layout), residual adds in the out / down epilogues, against the separate add+RMSNorm
    x = torch.randn(B, d, generator=g).to(dev)
    xt = K.tile_f32(x)
    gam = (1 + 0.1 * torch.randn(d, generator=g)).to(dev)
    rstd = torch.empty(B, device=dev)
    delta = torch.randn(B, d, generator=g).to(dev)
    xs = torch.empty(K.split_numel(B, d, True), device=dev, dtype=torch.bfloat16)
    res["add_rmsnorm_us"] = round(graph_time_us(
        lambda: K.add_rmsnorm(x, delta, None, gam, 1e-5, xs, rstd, tiled=True)), 2)
    for name, N, k in (("qkv", 3 * d, d), ("out", d, d), ("gate_up", 2 * F, d), ("down", d, F)):
        a = K.tile_matrix(torch.randn(B, 2 * k, generator=g).to(dev, torch.bfloat16))
        wt = K.tile_matrix((0.05 * torch.randn(N, k, generator=g)).to(dev, torch.bfloat16))
        if name == "qkv":
            out = torch.empty(B, N, device=dev)
            res[name]["k5_norm_us"] = round(graph_time_us(
                lambda: K.gemm_norm(xt, gam, 1e-5, wt, out, rstd, k)), 2)
        elif name == "gate_up":
            h = torch.empty(K.split_numel(B, F, True), device=dev, dtype=torch.bfloat16)
            res[name]["k5_norm_swiglu_us"] = round(graph_time_us(
                lambda: K.gemm_norm_swiglu(xt, gam, 1e-5, wt, None, None, h, B, F, k)), 2)
        else:
            xr = K.tile_f32(torch.zeros(B, N, device=dev))
            res[name]["k5_residual_us"] = round(graph_time_us(
                lambda: K.gemm_split_residual(a, wt, xr, None, B, N, k)), 2)
    res["per_layer_us"] = dict(
        hipblaslt_plus_swiglu=round(sum(res[n]["hipblaslt_us"] for n in
                                        ("qkv", "out", "gate_up", "down")) +
                                    res["gate_up"]["swiglu_us"], 2),
        k5_fused=round(res["qkv"]["k5_us"] + res["out"]["k5_us"] + res["down"]["k5_us"] +
                       res["gate_up"]["fused_swiglu_us"], 2),
        k5_fused_plus_2_add_rmsnorm=round(res["qkv"]["k5_us"] + res["out"]["k5_us"] +
                                          res["down"]["k5_us"] +
                                          res["gate_up"]["fused_swiglu_us"] +
                                          2 * res["add_rmsnorm_us"], 2),
        k5_norm_fused=round(res["qkv"]["k5_norm_us"] + res["out"]["k5_residual_us"] +
                            res["gate_up"]["k5_norm_swiglu_us"] +
                            res["down"]["k5_residual_us"], 2))
    return res


def augmentation_bench(model, dev, spec):
    """predict_with_augmentations (the caller of the path, src/inference.py:697-920) on one
    synthetic task of ``spec``: 64 prompts (8 dihedral x 8 colour permutations), greedy, the
    workload's decode budget.  Fused (one generation, per-row chunk semantics) against the chunk
    loop of 16 rows; wall seconds of one call each after a warm call, host prompt building and
    grid decoding included."""
    import torch

    from mdlarc_scale_amd import inference as I
    from mdlarc_scale_amd.workload import task_dict

    task = task_dict(spec)
    kw = dict(num_color_perms=8, max_output_tokens=spec.max_new)
    res = {}
    preds = {}
    for name, fuse in (("fused", True), ("chunks_of_16", False)):
        I.predict_with_augmentations(model, task, 0, dev, fuse_chunks=fuse, **kw)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        preds[name] = I.predict_with_augmentations(model, task, 0, dev, fuse_chunks=fuse, **kw)
        torch.cuda.synchronize()
        res[f"{name}_s"] = round(time.perf_counter() - t0, 4)
    n_tok = [len(v.tokens) for v in I._build_variants(task, 0, True, 8, 1, False, None, None)]
    res.update(variants=len(preds["fused"]), prompt_len_min=min(n_tok),
               prompt_len_max=max(n_tok), max_output_tokens=spec.max_new,
               speedup=round(res["chunks_of_16_s"] / res["fused_s"], 2),
               identical_predictions=preds["fused"] == preds["chunks_of_16"])
    return res


def snapshot_decode_state(st, ex):
    """Host copy of what the CPU baseline continues from: the cache (bf16 -> fp32), the current
    token, the grid state and the masks."""
    return dict(B=st.B, S=st.S, total=st.total, cache=st.cache.cache.cpu().float(),
                tok=st.tok.cpu(), gx=st.gx.cpu(), gy=st.gy.cpu(), gio=st.gio.cpu(),
                pmask=st.pmask.cpu().bool(), ex=ex.cpu())


def cpu_baseline(model_state, cfg, snap, t0, seconds):
    """fp32 CPU oracle decoding the same B rows from the GPU's cache contents (upcast to fp32)
    for as many steps as fit in ``seconds`` (at least 2)."""
    import torch

    from oracle import reference_path as rp

    ocfg = rp.OracleConfig(cfg.d_model, cfg.n_heads, cfg.n_layers, cfg.d_ff, cfg.num_examples,
                           cfg.max_seq_len)
    om = rp.OracleModel(ocfg, model_state, dtype=torch.float32)
    B, S, total = snap["B"], snap["S"], snap["total"]
    cache = snap["cache"]
    tok = snap["tok"]
    grid = rp.GridState(snap["gx"], snap["gy"], snap["gio"])
    key_mask = torch.ones(B, total, dtype=torch.bool)
    key_mask[:, :S] = snap["pmask"]
    exc = snap["ex"]
    steps, t = 0, t0
    start = time.perf_counter()
    while t + 1 < total:
        pos = grid.update(tok)
        logits = om.decode_step(tok, pos, exc, cache, t, key_mask[:, :t + 1])
        tok = logits.argmax(-1)
        steps += 1
        t += 1
        if time.perf_counter() - start >= seconds and steps >= 2:
            break
    el = time.perf_counter() - start
    return dict(value=round(B * steps / el, 2), unit="tokens/s", cores=torch.get_num_threads(),
                kind="port",
                sample=f"B={B} rows x {steps} greedy decode steps of the fp32 oracle "
                       f"(oracle/reference_path.py OracleModel.decode_step) from cache fill "
                       f"t={t0}, cache filled from the GPU prefill/decode K/V upcast to fp32; "
                       f"{el:.1f} s on {torch.get_num_threads()} threads "
                       f"({platform.processor() or platform.machine()}, "
                       f"os.cpu_count()={os.cpu_count()})")


def measure_workload(spec, steps, warmup, dev, eager=False, snapshot=False):
    """Prefill and ``steps`` timed greedy decode steps of ``spec``'s batch (after ``warmup``
    untimed ones), then the decode attention's timed launches re-issued under HIP events and one
    layer's prefill-attention launch re-issued 10 times.  Returns the measurements, plus the
    model and decode state when ``snapshot`` (the CPU baseline continues from them)."""
    import torch

    from mdlarc_scale_amd import kernels as K
    from mdlarc_scale_amd import inference as I
    from mdlarc_scale_amd.data import END_TOKEN_ID
    from mdlarc_scale_amd.engine import engine_for, pack_prompt
    from mdlarc_scale_amd.transformer import MODEL_SIZES, attention_q_scale, create_model
    from mdlarc_scale_amd.workload import build_prompts, left_pad

    t_build = time.perf_counter()
    prompts = build_prompts(spec)
    ids, pos, mask = left_pad(prompts)
    B, S = ids.shape
    per_task = spec.batch // spec.n_tasks
    ex = torch.arange(spec.n_tasks).repeat_interleave(per_task)
    host_build_s = time.perf_counter() - t_build

    torch.manual_seed(0)
    model = create_model(**MODEL_SIZES[spec.preset], dropout=0.0, max_seq_len=spec.cache_slots)
    model = model.to(torch.bfloat16)                 # bf16 models
    model_state = ({k: v.float().clone() for k, v in model.state_dict().items()}
                   if snapshot else None)
    model = model.to(dev).eval()
    cfg = model.config
    total = min(S + spec.max_new, cfg.max_seq_len)
    max_new = total - S
    if warmup + steps + 1 > max_new:
        raise SystemExit(f"--warmup + --steps = {warmup + steps} exceeds the {max_new - 1} decode "
                         f"steps the {cfg.max_seq_len}-slot cache leaves after the {S}-token "
                         f"prompts of {spec.name}")

    eng = engine_for(model)
    gen = I.Generator(model)
    ids_d, pos_d, mask_d, ex_d = ids.to(dev), pos.to(dev), mask.to(dev), ex.to(dev)
    res = {}
    with torch.no_grad():
        W = eng.packed(dev)
        st = gen.prepare(ids_d, pos_d, ex_d, mask_d, total)
        gen.prefill(st, W, ids_d, pos_d)       # warm (library setup, allocations); idempotent
        torch.cuda.synchronize()
        # the median of three prefills: one prefill is a single sample of a few to a few hundred
        # ms, whose box-to-box and run-to-run spread (about 1%) hides changes of that size
        samples = []
        for _ in range(3):
            tp = Timer()
            tp.start()
            gen.prefill(st, W, ids_d, pos_d)
            tp.stop()
            samples.append(tp.ms())
        prefill_ms = sorted(samples)[1]
        K.decode_commit(st.tok, st.out_ids, S, None, st.finish, S, END_TOKEN_ID)
        # warmup: one eager step, capture, replays
        gen.greedy_step(st, W, True)
        graph = None if eager else gen.capture_greedy(st, W, True)
        for _ in range(warmup - 1):
            graph.replay() if graph is not None else gen.greedy_step(st, W, True)
        torch.cuda.synchronize()
        t_first = S + warmup                   # cache slot of the first timed step's token
        tm = Timer()
        wall0 = time.perf_counter()
        tm.start()
        for _ in range(steps):
            graph.replay() if graph is not None else gen.greedy_step(st, W, True)
        tm.stop()
        torch.cuda.synchronize()
        wall_s = time.perf_counter() - wall0
        timed_ms = tm.ms()

        # the CPU baseline continues from this state; take it before the re-launches below
        # rewrite the slots they attend to
        snap = snapshot_decode_state(st, ex_d) if snapshot else None

        # decode attention (the mdl_attn_decode launch the step runs on the q the qkv
        # projection wrote): re-issue the timed region's launches (every layer at every cache
        # position t of the timed steps) back to back on the launching stream, between one pair
        # of HIP events; the queue never drains, so the events time kernel execution only
        H = cfg.n_heads
        kv_start_h, holes_h = st.kv_start.cpu(), st.holes.cpu()
        ts = [t_first + i for i in range(steps) for _ in range(cfg.n_layers)]
        layers = [li for _ in range(steps) for li in range(cfg.n_layers)]
        ta = Timer()
        ta.start()
        for t, li in zip(ts, layers):
            kc, vc = st.cache.layer(li)
            K.attn_decode(st.sc.q, kc, vc, B, H, st.pmask, S, st.kv_start, t, None, st.ws,
                          st.split_len, st.sc.attn, row_holes=st.holes, row_order=st.order,
                          tiled=st.sc.tiled)
        ta.stop()
        attn_ms = ta.ms() / len(ts)
        attn_bytes = sum(decode_attention_bytes(B, H, t, kv_start_h, S, holes_h)
                         for t in ts) / len(ts)
        # the launch's own choices (csrc/attn_decode.hip decode_impl): wave tiles of 64 slots
        # once a work item can exceed 2,048 slots, else 32; ceil(total / split_len) splits
        n_split = -(-total // st.split_len)
        decode_nb = 4 if min(st.split_len, total) > 2048 else 2

        # prefill attention alone: one layer's launch as the prefill makes it (packed query
        # rows) over the batch's own masks and cache, with synthetic q of unit-variance rows
        # pre-scaled as the projection scales q (the softmax scale times log2(e)); the kernel's
        # time depends on values only through how often a query's running maximum moves
        n_valid = mask.sum(1)
        pa_flops = 4 * 64 * H * int((n_valid * (n_valid + 1) // 2).sum())
        # its algorithmic HBM bytes: bf16 q, the K and V rows of every valid key once, the
        # hi|lo output, and the prompt-mask bytes of rows whose mask has holes
        pa_bytes = int(n_valid.sum()) * H * 64 * 2 * 5 + int(
            ((S - kv_start_h.to(torch.int64)).clamp(min=0) * holes_h.to(torch.int64)).sum())
        starts = torch.stack([st.kv_start, st.last_row]).cpu().numpy()
        pk = pack_prompt(starts[0], starts[1], B, S, dev)
        qp = (torch.randn(pk.n_valid, H * 64, device=dev)
              * attention_q_scale(64)).to(torch.bfloat16)
        op = torch.empty(pk.n_valid, 2 * H * 64, device=dev, dtype=torch.bfloat16)
        kc0, vc0 = st.cache.layer(0)

        def prefill_attention():
            K.attn_prefill_packed(qp, kc0, vc0, B, S, H, st.pmask, st.kv_start, pk.q_offset,
                                  pk.n_valid, True, op, row_holes=st.holes)

        # steady state: 3 warm launches, then the median of 5 rounds of 10 back-to-back launches
        for _ in range(3):
            prefill_attention()
        reps, rounds = 10, []
        for _ in range(5):
            tpa = Timer()
            tpa.start()
            for _ in range(reps):
                prefill_attention()
            tpa.stop()
            rounds.append(tpa.ms() / reps)
        pa_ms = sorted(rounds)[len(rounds) // 2]
        del qp, op

        # the prompt projections alone (K6): one layer's four launches as the prefill makes
        # them (pk.n_tokens rows, the layer-0 weights), on synthetic activations and a scratch
        # cache layer (the kernels' time does not depend on values); steady state as above
        proj = prefill_projections_timing(K, W, cfg, pk, st, dev) if W.tiles_ok else None

    res.update(
        B=B, S=S, total=total, max_new=max_new, t_first=t_first, host_build_s=host_build_s,
        prefill_ms=prefill_ms, timed_ms=timed_ms, wall_s=wall_s,
        value=B * steps / (timed_ms / 1e3), attn_ms=attn_ms, attn_bytes=attn_bytes,
        attn_launches=len(ts), n_split=n_split, decode_nb=decode_nb, n_valid=n_valid,
        pa_ms=pa_ms, pa_flops=pa_flops, pa_bytes=pa_bytes,
        prefill_flops=cfg.n_layers * pa_flops, snap=snap,
        proj=proj,
        model_state=model_state, cfg=cfg)
    if snapshot:
        res.update(model=model, st=st)
    return res


def prefill_projections_timing(K, W, cfg, pk, st, dev):
    """Milliseconds per launch of each K6 form of one prefill layer (median of 5 rounds of 5
    back-to-back launches after 2 warm ones) and its executed MFMA flops (2·parts·M·N·K: the hi
    and lo products of a split activation, the hi product alone for the MLP's single-part
    inputs), as the prompt path calls them."""
    import torch

    from mdlarc_scale_amd.engine import PROMPT_DOWN_PARTS as dp
    from mdlarc_scale_amd.engine import PROMPT_GATE_UP_PARTS as gp
    from mdlarc_scale_amd.engine import Scratch

    m, d, F, H = pk.n_tokens, cfg.d_model, cfg.d_ff, cfg.n_heads
    sc = Scratch.alloc(m, d, F, dev, fused=True)
    g = torch.Generator(device=dev).manual_seed(5)
    sc.x.normal_(generator=g)
    sc.attn.copy_(torch.randn(sc.attn.shape, generator=g, device=dev).to(torch.bfloat16))
    sc.h.copy_(torch.randn(sc.h.shape, generator=g, device=dev).to(torch.bfloat16))
    kc0, _ = st.cache.layer(0)
    kc, vc = torch.empty_like(kc0), torch.empty_like(kc0)
    pos = torch.zeros(m, 3, dtype=torch.int64, device=dev)
    qs = 1.0 / 8.0
    forms = {
        "qkv_rope": (4 * m * 3 * d * d, lambda: K.prefill_gemm_norm_qkv(
            sc.x, W.ln1[0], W.eps, W.qkv_t[0], m, H, sc.rstd, sc.qkv, K.LEAD_QUERIES,
            st.kv_start, pos, W.rope_tab, W.rope_geom, qs, sc.q, kc, vc,
            token_row=pk.token_row, token_slot=pk.token_slot)),
        "out_residual": (4 * m * d * d, lambda: K.prefill_gemm_split_residual(
            sc.attn, W.out_t[0], sc.x, None, m, d, d, a_tiled=True)),
        "gate_up_swiglu": (2 * gp * m * 2 * F * d, lambda: K.prefill_gemm_norm_swiglu(
            sc.x, W.ln2[0], W.eps, W.gu_t[0], W.b_gate[0], W.b_up[0], sc.h, m, F, d,
            a_parts=gp, h_parts=dp)),
        "down_residual": (2 * dp * m * d * F, lambda: K.prefill_gemm_split_residual(
            sc.h, W.down_t[0], sc.x, W.b_down[0], m, d, F, a_tiled=True, a_parts=dp)),
    }
    out = {}
    for name, (flops, fn) in forms.items():
        for _ in range(2):
            fn()
        rounds = []
        for _ in range(5):
            t = Timer()
            t.start()
            for _ in range(5):
                fn()
            t.stop()
            rounds.append(t.ms() / 5)
        out[name] = (sorted(rounds)[2], flops)
    del sc, kc, vc
    return out


def prefill_projections_of(r):
    """The prompt projections' MFMA rate (K6, one layer): executed flops over launch time."""
    proj = r.get("proj")
    if not proj:
        return None
    ms = sum(v[0] for v in proj.values())
    fl = sum(v[1] for v in proj.values())
    return {
        "kernel": "prefill_gemm_kernel (K6: mdl_prefill_gemm_norm_qkv, "
                  "mdl_prefill_gemm_split_residual x 2, mdl_prefill_gemm_norm_swiglu)",
        "bound": "mfma", "ms_per_layer": round(ms, 4), "tflop_per_layer": round(fl / 1e12, 4),
        "achieved": round(fl / ms / 1e9, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
        "frac": round(fl / ms / 1e9 / BF16_PEAK_TFLOPS, 4),
        "forms": {k: {"ms": round(v[0], 4), "tflop_s": round(v[1] / v[0] / 1e9, 1)}
                  for k, v in proj.items()},
        "flops": "executed bf16 MFMA flops, 2·parts·M·N·K per projection: the hi and lo "
                 "products of a split input (half of them useful), the hi product alone for a "
                 "single-part MLP input (engine.PROMPT_GATE_UP_PARTS / PROMPT_DOWN_PARTS)",
    }


def roofline_of(r):
    """The decode attention's roofline object: algorithmic bytes per launch over its average
    launch duration against the 8 TB/s peak."""
    achieved = r["attn_bytes"] / r["attn_ms"] / 1e6
    return {
        "kernel": f"attn_decode_kernel<false, {r['decode_nb']}> (mdl_attn_decode: decode "
                  f"attention on bf16 MFMA over the q and slot-t K/V that the qkv projection's "
                  f"epilogue wrote, {16 * r['decode_nb']}-slot wave tiles, {r['n_split']} "
                  f"split(s) per (row, head))",
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
        "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
        "avg_launch_ms": round(r["attn_ms"], 5), "bytes_per_launch": int(r["attn_bytes"]),
        "launches_timed": r["attn_launches"],
    }


def prefill_attention_of(r):
    pa_ms, pa_flops = r["pa_ms"], r["pa_flops"]
    out = {
        "kernel": "attn_prefill_kernel (mdl_attn_prefill_packed, bf16 MFMA)", "bound": "mfma",
        "ms_per_layer": round(pa_ms, 4), "tflop_per_layer": round(pa_flops / 1e12, 4),
        "achieved": round(pa_flops / pa_ms / 1e9, 1), "peak": BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s", "frac": round(pa_flops / pa_ms / 1e9 / BF16_PEAK_TFLOPS, 4),
        "flops": "valid causal (query, key) pairs x 4 x 64 (QK^T and PV)",
    }
    if r.get("pa_bytes"):
        # the same launches against the HBM roofline (the rocprofv3 FETCH_SIZE / WRITE_SIZE
        # passes measure 1.02-1.04 / 1.00 of these bytes)
        gbs = r["pa_bytes"] / pa_ms / 1e6
        out["hbm"] = {"bytes_per_launch": r["pa_bytes"], "achieved": round(gbs, 1),
                      "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                      "bytes": "bf16 q, the K and V rows of every valid key once, the hi|lo "
                               "output, prompt-mask bytes of rows with holes",
                      "traffic_source": "profiles/prefill_attention_mfma.md"}
    return out


def prefill_of(r):
    nv = int(r["n_valid"].sum())
    return {"ms": round(r["prefill_ms"], 3), "tokens": nv, "padded_tokens": r["B"] * r["S"],
            "tokens_per_s": round(nv / (r["prefill_ms"] / 1e3), 1),
            "attention_causal_tflop": round(r["prefill_flops"] / 1e12, 3)}


def side_config(name, dev, steps=32, warmup=4):
    """BASELINE configs 3 and 4 on the default line: decode tokens/s over ``steps`` graph-replayed
    steps, the decode attention's GB/s, the prefill and one layer's prefill-attention TFLOP/s."""
    import torch

    from mdlarc_scale_amd.workload import SPECS

    r = measure_workload(SPECS[name], steps, warmup, dev)
    out = {
        "workload": WORKLOADS[name], "rows": r["B"], "padded_prompt_slots": r["S"],
        "cache_slots": r["total"], "prompt_len_min": int(r["n_valid"].min()),
        "prompt_len_max": int(r["n_valid"].max()), "steps": steps, "warmup": warmup,
        "decode_tokens_per_s": round(r["value"], 1),
        "ms_per_step": round(r["timed_ms"] / steps, 4),
        "timed_cache_fill": [r["t_first"], r["t_first"] + steps],
        "decode_attention": roofline_of(r), "prefill": prefill_of(r),
        "prefill_attention": prefill_attention_of(r),
        "prefill_projections": prefill_projections_of(r),
    }
    del r
    return out


def main() -> int:
    args = _args()
    if args.gpus != 1:
        print("bench.py runs on exactly one GPU: this build measures the single-GPU hot path "
              "(decode rows would shard by batch across GPUs with no exchange, so one GPU's "
              "throughput is the per-GPU figure). Use --gpus 1.", file=sys.stderr)
        return 2
    import torch

    from mdlarc_scale_amd import _lib
    from mdlarc_scale_amd.workload import SPECS

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    _lib.lib()
    dev = torch.device("cuda:0")
    spec = SPECS[args.config]
    headline = spec.name == "small_b256"
    if args.cpu_seconds is None:
        args.cpu_seconds = 15.0 if headline else 0.0
    r = measure_workload(spec, args.steps, args.warmup, dev, eager=args.eager,
                         snapshot=args.cpu_seconds > 0 or args.augment or args.gemm_compare)
    cfg, B, S = r["cfg"], r["B"], r["S"]
    with torch.no_grad():
        micro = None if (args.no_micro or not headline) else microbench(dev)
        gemm_cmp = decode_gemm_compare(cfg, B, dev) if args.gemm_compare else None
        augment = augmentation_bench(r["model"], dev, spec) if args.augment else None
        cpu = None
        if args.cpu_seconds > 0:
            cpu = cpu_baseline(r["model_state"], cfg, r["snap"],
                               S + args.warmup + args.steps, args.cpu_seconds)
    r.pop("snap", None)
    r.pop("model", None)
    r.pop("st", None)
    # no torch.cuda.empty_cache() between configurations: returning cached memory to the driver
    # leaves later HBM-bound kernels of the process slower (see Generator.capture_greedy)
    sides = {}
    if headline and not args.no_side:
        for name in ("medium_b128", "large_b64"):
            sides[name] = side_config(name, dev)

    roof = roofline_of(r)
    ratio, traffic_src = recorded_traffic_ratio("attn_decode_kernel", spec.name)
    roof["traffic"] = None if ratio is None else int(round(ratio * roof["bytes_per_launch"]))
    roof["traffic_per_algorithmic_byte"] = ratio
    roof["traffic_source"] = traffic_src
    n_valid = r["n_valid"]
    out = {
        "metric": METRIC if headline else f"greedy decode tokens/s at {spec.preset}, B={B}",
        "value": round(r["value"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["timed_ms"] / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": WORKLOADS[spec.name],
            "preset": spec.preset, "rows": B, "padded_prompt_slots": S,
            "cache_slots": r["total"], "decode_steps_available": r["max_new"] - 1,
            "timed_cache_fill": [r["t_first"], r["t_first"] + args.steps],
            "prompt_len_min": int(n_valid.min()), "prompt_len_mean": round(float(
                n_valid.float().mean()), 1), "prompt_len_max": int(n_valid.max()),
            "sharding": "one GPU (rows would shard by batch across GPUs, no exchange)",
            "graph": not args.eager, "workload_seed": spec.seed,
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "prefill": prefill_of(r),
        "prefill_attention": prefill_attention_of(r),
        "prefill_projections": prefill_projections_of(r),
        "microbench": micro,
        **({"configs": sides} if sides else {}),
        **({"augmentation": augment} if augment is not None else {}),
        **({"decode_gemm": gemm_cmp} if gemm_cmp is not None else {}),
        "wall_s_timed": round(r["wall_s"], 4),
        "host_prompt_build_s": round(r["host_build_s"], 3),
    }
    if cpu:
        out["vs_cpu"] = round(r["value"] / cpu["value"], 1)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
