"""Kernel-level parity on the GPU: every entry point of libmdlarc_hip.so, called through the C ABI
(mdlarc_scale_amd.kernels), against the CPU oracle on identical seeded inputs.

Tolerances: values the kernel rounds to one bf16 are compared at bf16 resolution
(|a-b| <= 1e-2*|b| + atol); split (hi|lo bf16) outputs are recombined and compared at about
2^-16 relative; fp32 outputs at fp32 resolution; integer outputs exactly.
"""

import math

import numpy as np
import pytest
import torch

from mdlarc_scale_amd.transformer import LOG2E
from oracle import reference_path as rp

pytestmark = pytest.mark.gpu

DEV = "cuda"


def K():
    from mdlarc_scale_amd import kernels

    return kernels


def bf(t):
    return t.to(torch.bfloat16)


def close_bf16(got, ref, atol=1e-3, rtol=1e-2):
    got, ref = got.float().cpu(), ref.float().cpu()
    err = (got - ref).abs()
    bound = atol + rtol * ref.abs()
    assert bool((err <= bound).all()), f"max err {err.max().item():.3e}, worst ratio " \
        f"{(err / bound).max().item():.2f}"


def _cfg(d, H):
    return rp.OracleConfig(d_model=d, n_heads=H, n_layers=1, d_ff=64)


def unsplit(t):
    """[rows, 2K] hi|lo bf16 -> [rows, K] fp32 (hi + lo)."""
    t = t.float().cpu()
    k = t.shape[-1] // 2
    return t[..., :k] + t[..., k:]


def check_split(t, ref, rtol=2e-5, atol=1e-7):
    """hi is the bf16 rounding of the value (to 1 ulp of the kernel's fp32 arithmetic) and
    hi + lo equals it to about 2^-16 relative."""
    t = t.cpu()
    k = t.shape[-1] // 2
    hi = t[..., :k].float()
    ref = ref.float()
    assert torch.allclose(hi, ref.to(torch.bfloat16).float(), rtol=8e-3, atol=atol)
    got = unsplit(t)
    err = (got - ref).abs()
    bound = atol + rtol * ref.abs()
    assert bool((err <= bound).all()), f"split max err {err.max().item():.3e}"


# ---------------------------------------------------------------------------- K1 / add_rmsnorm

@pytest.mark.parametrize("d", [128, 256, 768, 1280])
@pytest.mark.parametrize("table_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_ex", [True, False])
def test_embed_rmsnorm(d, table_dtype, with_ex):
    g = torch.Generator().manual_seed(d)
    B, S, V, NE = 3, 37, 14, 5
    tok = torch.randn(V, d, generator=g).to(table_dtype)
    ex = torch.randn(NE, d, generator=g).to(table_dtype)
    ids = torch.randint(0, V, (B, S), generator=g)
    ex_ids = torch.randint(0, NE, (B,), generator=g)
    gamma = 1 + 0.1 * torch.randn(d, generator=g)
    x_ref = tok.float()[ids] + (ex.float()[ex_ids][:, None] if with_ex else 0)
    x_ref = x_ref.reshape(B * S, d)
    r_ref = torch.rsqrt((x_ref.double() ** 2).mean(-1) + 1e-5).float()
    x = torch.empty(B * S, d, device=DEV)
    xs = torch.empty(B * S, 2 * d, device=DEV, dtype=torch.bfloat16)
    r = torch.empty(B * S, device=DEV)
    K().embed_rmsnorm(ids.to(DEV).reshape(-1), ex_ids.to(DEV) if with_ex else None, tok.to(DEV),
                      ex.to(DEV) if with_ex else None, S, gamma.to(DEV), 1e-5, x, xs, r)
    torch.cuda.synchronize()
    assert torch.allclose(x.cpu(), x_ref, atol=1e-6, rtol=1e-6)
    assert torch.allclose(r.cpu(), r_ref, rtol=2e-6)
    check_split(xs, x_ref.double() * gamma.double())


@pytest.mark.parametrize("d", [128, 768, 800])
@pytest.mark.parametrize("with_ex", [True, False])
def test_embed_rmsnorm_bf16(d, with_ex):
    """Config-1 format of K1: x is the bf16 rounding of the fp32 sum of the two bf16 rows
    (exactly what a bf16 model's embedding add gives); xn = x * rstd * gamma from the rounded x,
    against fp64 at bf16 resolution."""
    g = torch.Generator().manual_seed(d + 1)
    B, S, V, NE = 3, 37, 14, 5
    tok = torch.randn(V, d, generator=g).to(torch.bfloat16)
    ex = torch.randn(NE, d, generator=g).to(torch.bfloat16)
    ids = torch.randint(0, V, (B, S), generator=g)
    ex_ids = torch.randint(0, NE, (B,), generator=g)
    gamma = 1 + 0.1 * torch.randn(d, generator=g)
    x_ref = (tok.float()[ids] + (ex.float()[ex_ids][:, None] if with_ex else 0)).reshape(B * S, d)
    x_ref = x_ref.to(torch.bfloat16)
    xd = x_ref.double()
    xn_ref = xd * torch.rsqrt((xd ** 2).mean(-1, keepdim=True) + 1e-5) * gamma.double()
    x = torch.empty(B * S, d, device=DEV, dtype=torch.bfloat16)
    xn = torch.empty_like(x)
    K().embed_rmsnorm_bf16(ids.to(DEV).reshape(-1), ex_ids.to(DEV) if with_ex else None,
                           tok.to(DEV), ex.to(DEV) if with_ex else None, S, gamma.to(DEV), 1e-5,
                           x, xn)
    torch.cuda.synchronize()
    assert torch.equal(x.cpu(), x_ref)
    close_bf16(xn, xn_ref.float(), atol=1e-6, rtol=8e-3)


@pytest.mark.parametrize("d", [256, 768, 1024])
def test_add_rmsnorm(d):
    g = torch.Generator().manual_seed(7)
    M = 129
    x0 = torch.randn(M, d, generator=g)
    delta = torch.randn(M, d, generator=g)
    bias = 0.1 * torch.randn(d, generator=g)
    gamma = 1 + 0.1 * torch.randn(d, generator=g)
    for use_delta, use_bias, use_xs in ((True, True, True), (True, False, True),
                                        (False, False, False)):
        x = x0.to(DEV).clone()
        xs = torch.empty(M, 2 * d, device=DEV, dtype=torch.bfloat16) if use_xs else None
        r = torch.empty(M, device=DEV)
        K().add_rmsnorm(x, delta.to(DEV) if use_delta else None, bias.to(DEV) if use_bias else None,
                        gamma.to(DEV), 1e-5, xs, r)
        torch.cuda.synchronize()
        ref = x0 + (delta if use_delta else 0) + (bias if use_bias else 0)
        assert torch.allclose(x.cpu(), ref, atol=1e-6)
        assert torch.allclose(r.cpu(), torch.rsqrt(ref.pow(2).mean(-1) + 1e-5), rtol=2e-6)
        if use_xs:
            check_split(xs, ref.double() * gamma.double())


# ---------------------------------------------------------------------------- K2

@pytest.mark.parametrize("H,S,slot0", [(2, 1, 5), (4, 33, 0), (12, 64, 10), (16, 5, 3),
                                        (20, 7, 100)])
def test_qkv_rope_cache(H, S, slot0):
    d = 64 * H
    B, slots = 3, 200
    cfg = _cfg(d, H)
    g = torch.Generator().manual_seed(H * 100 + S)
    qkv = torch.randn(B * S, 3 * d, generator=g)
    rstd = 0.5 + torch.rand(B * S, generator=g)
    pos = torch.randint(-3, 40, (B * S, 3), generator=g)
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    rope = RotaryEmbedding3D(64, cfg.max_x, cfg.max_y, cfg.max_z)
    tab = rope.device_table(DEV)
    geom = (rope.max_x, rope.max_y, rope.max_z, rope.px, rope.py, rope.pz)
    q = torch.empty(B * S, d, device=DEV, dtype=torch.bfloat16)
    kc = torch.full((B, H, slots, 64), 7.0, device=DEV, dtype=torch.bfloat16)
    vc = torch.full_like(kc, 7.0)
    K().qkv_rope_cache(qkv.to(DEV), rstd.to(DEV), pos.to(DEV), tab, geom, B, S, H, 0.125, q, kc,
                       vc, slot0=slot0)
    torch.cuda.synchronize()
    y = (qkv.float() * rstd[:, None]).view(B, S, 3, H, 64)
    tabs = rp.rope3d_tables(cfg)
    p3 = pos.view(B, S, 3)
    q_ref = rp.apply_rope3d(y[:, :, 0], p3, tabs, cfg) * 0.125
    k_ref = rp.apply_rope3d(y[:, :, 1], p3, tabs, cfg)
    close_bf16(q.view(B, S, H, 64), q_ref)
    close_bf16(kc[:, :, slot0:slot0 + S].permute(0, 2, 1, 3), k_ref)
    close_bf16(vc[:, :, slot0:slot0 + S].permute(0, 2, 1, 3), y[:, :, 2])
    untouched = torch.ones(slots, dtype=torch.bool)
    untouched[slot0:slot0 + S] = False
    assert bool((kc[:, :, untouched.to(DEV)] == 7).all())
    assert bool((vc[:, :, untouched.to(DEV)] == 7).all())


@pytest.mark.parametrize("H,S,slot0,with_rstd", [(4, 33, 0, True), (12, 64, 10, True),
                                                   (16, 5, 3, False), (20, 7, 100, True)])
def test_qkv_rope_cache_bf16(H, S, slot0, with_rstd):
    """Config-1 format of K2 (bf16 qkv in) against the oracle's 3D RoPE on the same bf16
    values, at bf16 resolution; cache slots outside [slot0, slot0 + S) untouched."""
    d = 64 * H
    B, slots = 3, 200
    cfg = _cfg(d, H)
    g = torch.Generator().manual_seed(H * 100 + S + 1)
    qkv = torch.randn(B * S, 3 * d, generator=g).to(torch.bfloat16)
    rstd = 0.5 + torch.rand(B * S, generator=g)
    pos = torch.randint(-3, 40, (B * S, 3), generator=g)
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    rope = RotaryEmbedding3D(64, cfg.max_x, cfg.max_y, cfg.max_z)
    tab = rope.device_table(DEV)
    geom = (rope.max_x, rope.max_y, rope.max_z, rope.px, rope.py, rope.pz)
    q = torch.empty(B * S, d, device=DEV, dtype=torch.bfloat16)
    kc = torch.full((B, H, slots, 64), 7.0, device=DEV, dtype=torch.bfloat16)
    vc = torch.full_like(kc, 7.0)
    K().qkv_rope_cache_bf16(qkv.to(DEV), rstd.to(DEV) if with_rstd else None, pos.to(DEV), tab,
                            geom, B, S, H, 0.125, q, kc, vc, slot0=slot0)
    torch.cuda.synchronize()
    r = rstd[:, None] if with_rstd else 1.0
    y = (qkv.double() * r).view(B, S, 3, H, 64)
    tabs = rp.rope3d_tables(cfg)
    p3 = pos.view(B, S, 3)
    q_ref = rp.apply_rope3d(y[:, :, 0], p3, tabs, cfg) * 0.125
    k_ref = rp.apply_rope3d(y[:, :, 1], p3, tabs, cfg)
    close_bf16(q.view(B, S, H, 64), q_ref.float())
    close_bf16(kc[:, :, slot0:slot0 + S].permute(0, 2, 1, 3), k_ref.float())
    close_bf16(vc[:, :, slot0:slot0 + S].permute(0, 2, 1, 3), y[:, :, 2].float())
    untouched = torch.ones(slots, dtype=torch.bool)
    untouched[slot0:slot0 + S] = False
    assert bool((kc[:, :, untouched.to(DEV)] == 7).all())
    assert bool((vc[:, :, untouched.to(DEV)] == 7).all())


@pytest.mark.parametrize("H", [2, 4])       # generic kernel, whole-row kernel
def test_qkv_rope_cache_device_slot(H):
    B, slots = 4, 50
    d = 64 * H
    qkv = torch.randn(B, 3 * d).to(DEV)
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    rope = RotaryEmbedding3D(64, 32, 32, 8)
    geom = (32, 32, 8, rope.px, rope.py, rope.pz)
    pos = torch.randint(0, 30, (B, 3)).to(DEV)
    slot = torch.tensor([17], dtype=torch.int32, device=DEV)
    outs = []
    for mode in ("host", "dev"):
        q = torch.empty(B, d, device=DEV, dtype=torch.bfloat16)
        kc = torch.zeros(B, H, slots, 64, device=DEV, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        if mode == "host":
            K().qkv_rope_cache(qkv, None, pos, rope.device_table(DEV), geom, B, 1, H, 0.125, q, kc,
                               vc, slot0=17)
        else:
            K().qkv_rope_cache(qkv, None, pos, rope.device_table(DEV), geom, B, 1, H, 0.125, q, kc,
                               vc, slot0=0, slot_dev=slot)
        outs.append((q, kc, vc))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert bool(outs[1][1][:, :, 17].abs().sum() > 0)


# ---------------------------------------------------------------------------- K3

@pytest.mark.parametrize("F", [192, 704, 2048, 3392])
def test_swiglu(F):
    g = torch.Generator().manual_seed(F)
    M = 77
    gu = 3 * torch.randn(M, 2 * F, generator=g)
    r = 0.5 + torch.rand(M, generator=g)
    bg = 0.1 * torch.randn(F, generator=g)
    bu = 0.1 * torch.randn(F, generator=g)
    h = torch.empty(M, 2 * F, device=DEV, dtype=torch.bfloat16)
    K().swiglu(gu.to(DEV), r.to(DEV), bg.to(DEV), bu.to(DEV), h)
    torch.cuda.synchronize()
    a = gu[:, :F].double() * r[:, None].double() + bg.double()
    b = gu[:, F:].double() * r[:, None].double() + bu.double()
    check_split(h, rp.silu(a) * b, rtol=1e-5, atol=1e-6)
    h2 = torch.empty_like(h)
    K().swiglu(gu.to(DEV), None, None, None, h2)
    torch.cuda.synchronize()
    check_split(h2, rp.silu(gu[:, :F].double()) * gu[:, F:].double(), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("F,M", [(192, 77), (2048, 77), (3392, 5)])
def test_swiglu_bf16(F, M):
    """Config-1 format of K3: bf16 gate|up in, one bf16 h out, against the fp64 closed form at
    bf16 resolution, with and without rstd and biases."""
    g = torch.Generator().manual_seed(F + 2)
    gu = (3 * torch.randn(M, 2 * F, generator=g)).to(torch.bfloat16)
    r = 0.5 + torch.rand(M, generator=g)
    bg = 0.1 * torch.randn(F, generator=g)
    bu = 0.1 * torch.randn(F, generator=g)
    h = torch.empty(M, F, device=DEV, dtype=torch.bfloat16)
    K().swiglu_bf16(gu.to(DEV), r.to(DEV), bg.to(DEV), bu.to(DEV), h)
    h2 = torch.empty_like(h)
    K().swiglu_bf16(gu.to(DEV), None, None, None, h2)
    torch.cuda.synchronize()
    gd = gu.double()
    a = gd[:, :F] * r[:, None].double() + bg.double()
    b = gd[:, F:] * r[:, None].double() + bu.double()
    close_bf16(h, (rp.silu(a) * b).float(), atol=1e-5, rtol=8e-3)
    close_bf16(h2, (rp.silu(gd[:, :F]) * gd[:, F:]).float(), atol=1e-5, rtol=8e-3)


# ---------------------------------------------------------------------------- streaming paths

def test_streaming_paths_bit_identical():
    """Batches of 64 MiB or more go through the non-temporal load/store instantiations of K1,
    add+RMSNorm, K2 and K3.  The cache hint cannot change arithmetic: the first rows of a large
    batch must equal, bit for bit, the same rows run as a small (default-policy) batch."""
    g = torch.Generator(device=DEV).manual_seed(5)
    d, H, F, V, NE = 768, 12, 2048, 14, 9
    big, small = 12_288, 37                       # K1 at d=768: 12288*768*8 B = 75 MB

    def both(run):
        outs = [run(n) for n in (big, small)]
        torch.cuda.synchronize()
        for ob, os_ in zip(*outs):
            assert torch.equal(ob[:os_.shape[0]], os_)

    tok = torch.randn(V, d, device=DEV, generator=g).to(torch.bfloat16)
    ex = torch.randn(NE, d, device=DEV, generator=g).to(torch.bfloat16)
    gamma = 1 + 0.1 * torch.randn(d, device=DEV, generator=g)
    ids = torch.randint(0, V, (big,), device=DEV, generator=g)
    ex_ids = torch.randint(0, NE, (big,), device=DEV, generator=g)

    def k1(n):
        x = torch.empty(n, d, device=DEV)
        xs = torch.empty(n, 2 * d, device=DEV, dtype=torch.bfloat16)
        r = torch.empty(n, device=DEV)
        K().embed_rmsnorm(ids[:n], ex_ids[:n], tok, ex, 1, gamma, 1e-5, x, xs, r)
        return x, xs, r
    both(k1)

    x0 = torch.randn(big, d, device=DEV, generator=g)
    delta = torch.randn(big, d, device=DEV, generator=g)
    bias = 0.1 * torch.randn(d, device=DEV, generator=g)

    def add(n):
        x = x0[:n].clone()
        xs = torch.empty(n, 2 * d, device=DEV, dtype=torch.bfloat16)
        r = torch.empty(n, device=DEV)
        K().add_rmsnorm(x, delta[:n], bias, gamma, 1e-5, xs, r)
        return x, xs, r
    both(add)

    gu = torch.randn(big, 2 * F, device=DEV, generator=g)
    rs = 0.5 + torch.rand(big, device=DEV, generator=g)
    bg = 0.1 * torch.randn(F, device=DEV, generator=g)

    def k3(n):
        h = torch.empty(n, 2 * F, device=DEV, dtype=torch.bfloat16)
        K().swiglu(gu[:n], rs[:n], bg, bg, h)
        return (h,)
    both(k3)

    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    rope = RotaryEmbedding3D(64, 32, 32, 8)
    geom = (32, 32, 8, rope.px, rope.py, rope.pz)
    qkv = torch.randn(big, 3 * d, device=DEV, generator=g)
    pos = torch.randint(0, 30, (big, 3), device=DEV, generator=g)

    def k2(n):                                    # one row of n tokens: cache [1, H, n, 64]
        q = torch.empty(n, d, device=DEV, dtype=torch.bfloat16)
        kc = torch.zeros(1, H, n, 64, device=DEV, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        K().qkv_rope_cache(qkv[:n], rs[:n], pos[:n], rope.device_table(DEV), geom, 1, n, H,
                           0.125, q, kc, vc, slot0=0)
        return q, kc[0].transpose(0, 1), vc[0].transpose(0, 1)
    both(k2)

    # the config-1 (bf16 in and out) forms: K2 and K3 stream above 64 MiB at these sizes, K1's
    # two bf16 outputs from 21,846 rows of 768 channels on
    qkvb = qkv.to(torch.bfloat16)

    def k2b(n):
        q = torch.empty(n, d, device=DEV, dtype=torch.bfloat16)
        kc = torch.zeros(1, H, n, 64, device=DEV, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        K().qkv_rope_cache_bf16(qkvb[:n], rs[:n], pos[:n], rope.device_table(DEV), geom, 1, n,
                                H, 0.125, q, kc, vc, slot0=0)
        return q, kc[0].transpose(0, 1), vc[0].transpose(0, 1)
    both(k2b)
    gub = gu.to(torch.bfloat16)

    def k3b(n):
        h = torch.empty(n, F, device=DEV, dtype=torch.bfloat16)
        K().swiglu_bf16(gub[:n], rs[:n], bg, bg, h)
        return (h,)
    both(k3b)
    big = 24_576
    ids2 = torch.randint(0, V, (big,), device=DEV, generator=g)

    def k1b(n):
        x = torch.empty(n, d, device=DEV, dtype=torch.bfloat16)
        xn = torch.empty_like(x)
        K().embed_rmsnorm_bf16(ids2[:n], ex_ids[:1], tok, ex, n, gamma, 1e-5, x, xn)
        return x, xn
    both(k1b)


# ---------------------------------------------------------------------------- K4a prefill

def _masks(B, S, kind, g):
    m = torch.ones(B, S, dtype=torch.bool)
    if kind == "left":
        for b in range(B):
            n = int(torch.randint(0, S + 1, (1,), generator=g)) if b else S
            m[b, :S - n] = False
    elif kind == "holes":
        m = torch.rand(B, S, generator=g) < 0.7
    return m


@pytest.mark.parametrize("S", [1, 37, 64, 130, 257])
@pytest.mark.parametrize("kind", ["none", "left", "holes"])
@pytest.mark.parametrize("causal", [True, False])
def test_attn_prefill(S, kind, causal):
    g = torch.Generator().manual_seed(S * 7 + len(kind) + causal)
    B, H, slots = 3, 2, S + 9
    # q as the producers write it for the attention kernels: times the softmax scale 1/8 and
    # log2(e) (base-2 softmax); the reference undoes both
    q = bf(torch.randn(B, S, H, 64, generator=g) * 0.125)
    kc = bf(torch.randn(B, H, slots, 64, generator=g))
    vc = bf(torch.randn(B, H, slots, 64, generator=g))
    mask = _masks(B, S, kind, g) if kind != "none" else None
    kv_start = None
    if mask is not None:
        first = torch.where(mask.any(1), mask.float().argmax(1), torch.full((B,), S))
        kv_start = first.to(torch.int32).to(DEV)
    out = torch.empty(B * S, 2 * H * 64, device=DEV, dtype=torch.bfloat16)
    K().attn_prefill(q.to(DEV), kc.to(DEV), vc.to(DEV), B, S, H,
                     None if mask is None else mask.to(torch.uint8).to(DEV), kv_start, causal, out)
    torch.cuda.synchronize()
    ref = rp.attention((q.float() * 8 / LOG2E).transpose(1, 2), kc[:, :, :S].float(),
                       vc[:, :, :S].float(),
                       mask, causal)
    # P is rounded to bf16 for the PV MFMA: bf16-level agreement
    close_bf16(unsplit(out).view(B, S, H, 64).transpose(1, 2), ref, atol=8e-3, rtol=2e-2)


@pytest.mark.parametrize("causal", [True, False])
def test_attn_prefill_many_heads(causal):
    """B*H = 35 heads (several rounds of the 8-XCD block order, with padding blocks) over
    S = 700: six query tiles, ragged left padding, holes in one row, one row with no key."""
    g = torch.Generator().manual_seed(700 + causal)
    B, H, S, slots = 7, 5, 700, 768
    q = bf(torch.randn(B, S, H, 64, generator=g) * 0.125)
    kc = bf(torch.randn(B, H, slots, 64, generator=g))
    vc = bf(torch.randn(B, H, slots, 64, generator=g))
    mask = torch.ones(B, S, dtype=torch.bool)
    for b, n in enumerate([700, 1, 63, 64, 129, 450, 0]):
        mask[b, :S - n] = False
    mask[4, 600:611] = False
    first = torch.where(mask.any(1), mask.float().argmax(1), torch.full((B,), S))
    out = torch.empty(B * S, 2 * H * 64, device=DEV, dtype=torch.bfloat16)
    K().attn_prefill(q.to(DEV), kc.to(DEV), vc.to(DEV), B, S, H, mask.to(torch.uint8).to(DEV),
                     first.to(torch.int32).to(DEV), causal, out)
    torch.cuda.synchronize()
    ref = rp.attention((q.float() * 8 / LOG2E).transpose(1, 2), kc[:, :, :S].float(),
                       vc[:, :, :S].float(),
                       mask, causal)
    close_bf16(unsplit(out).view(B, S, H, 64).transpose(1, 2), ref, atol=8e-3, rtol=2e-2)


def test_attn_prefill_kv_start_clamped():
    """kv_start values outside [0, S] act as 0 (every key) and S (no key), never as addresses."""
    g = torch.Generator().manual_seed(91)
    B, H, S, slots = 3, 2, 150, 160
    q = bf(torch.randn(B, S, H, 64, generator=g) * 0.125)
    kc = bf(torch.randn(B, H, slots, 64, generator=g))
    vc = bf(torch.randn(B, H, slots, 64, generator=g))
    kv = torch.tensor([-1000, 10_000, 5], dtype=torch.int32)
    out = torch.empty(B * S, 2 * H * 64, device=DEV, dtype=torch.bfloat16)
    K().attn_prefill(q.to(DEV), kc.to(DEV), vc.to(DEV), B, S, H, None, kv.to(DEV), True, out)
    torch.cuda.synchronize()
    mask = torch.ones(B, S, dtype=torch.bool)
    mask[1] = False
    mask[2, :5] = False
    ref = rp.attention((q.float() * 8 / LOG2E).transpose(1, 2), kc[:, :, :S].float(),
                       vc[:, :, :S].float(),
                       mask, True)
    close_bf16(unsplit(out).view(B, S, H, 64).transpose(1, 2), ref, atol=8e-3, rtol=2e-2)


def _pack(kv, B, S):
    from mdlarc_scale_amd.engine import pack_prompt

    lengths = S - np.asarray(kv)
    last = np.arange(B) * S + np.maximum(lengths - 1, 0)
    return pack_prompt(np.asarray(kv), last, B, S, torch.device(DEV))


@pytest.mark.parametrize("H", [4, 12, 5])        # whole-row kernels and the per-head kernel
def test_qkv_rope_cache_packed_equals_padded(H):
    """The packed list (each row from its first valid token, plus the padding tokens that the
    lengths-1 index names) writes the q rows and cache slots the padded launch writes for those
    tokens, bit for bit, and no slot before a row's start."""
    d, S, slots = 64 * H, 37, 48
    kv = [0, 20, 37, 5]
    B = len(kv)
    g = torch.Generator().manual_seed(H)
    qkv = torch.randn(B * S, 3 * d, generator=g).to(DEV)
    rstd = (0.5 + torch.rand(B * S, generator=g)).to(DEV)
    pos = torch.randint(0, 31, (B * S, 3), generator=g).to(DEV)
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    rope = RotaryEmbedding3D(64, 32, 32, 8)
    tab, geom = rope.device_table(DEV), (32, 32, 8, rope.px, rope.py, rope.pz)
    q_pad = torch.empty(B * S, d, device=DEV, dtype=torch.bfloat16)
    kc_pad = torch.full((B, H, slots, 64), 7.0, device=DEV, dtype=torch.bfloat16)
    vc_pad = torch.full_like(kc_pad, 7.0)
    K().qkv_rope_cache(qkv, rstd, pos, tab, geom, B, S, H, 0.125, q_pad, kc_pad, vc_pad)
    pk = _pack(kv, B, S)
    gi = pk.gather.long()
    q_pk = torch.empty(pk.n_tokens, d, device=DEV, dtype=torch.bfloat16)
    kc_pk = torch.full_like(kc_pad, 7.0)
    vc_pk = torch.full_like(kc_pad, 7.0)
    K().qkv_rope_cache_packed(qkv[gi].contiguous(), rstd[gi].contiguous(), pos[gi].contiguous(),
                              tab, geom, pk.token_row, pk.token_slot, H, 0.125, q_pk, kc_pk,
                              vc_pk)
    torch.cuda.synchronize()
    assert pk.n_tokens == pk.n_valid + 2          # rows 1 and 2 read inside their padding
    assert torch.equal(q_pk, q_pad[gi])
    for b, k0 in enumerate(kv):
        assert torch.equal(kc_pk[b, :, k0:S], kc_pad[b, :, k0:S])
        assert torch.equal(vc_pk[b, :, k0:S], vc_pad[b, :, k0:S])
        assert bool((kc_pk[b, :, :k0] == 7).all()) and bool((vc_pk[b, :, :k0] == 7).all())
        assert bool((kc_pk[b, :, S:] == 7).all()) and bool((vc_pk[b, :, S:] == 7).all())


@pytest.mark.parametrize("causal", [True, False])
def test_attn_prefill_packed_equals_padded(causal):
    """Packed query rows give the padded launch's outputs for every query at or after its row's
    start, bit for bit; cache slots before a row's start hold NaN and never reach a product; no
    row outside the packed range is written."""
    g = torch.Generator().manual_seed(31 + causal)
    B, H, S, slots = 6, 3, 300, 320
    q = bf(torch.randn(B, S, H, 64, generator=g) * 0.125).to(DEV)
    kc = bf(torch.randn(B, H, slots, 64, generator=g)).to(DEV)
    vc = bf(torch.randn(B, H, slots, 64, generator=g)).to(DEV)
    kv = [0, 299, 170, 300, 64, 1]
    mask = torch.ones(B, S, dtype=torch.bool)
    for b, k0 in enumerate(kv):
        mask[b, :k0] = False
    mask[4, 200:230] = False                       # holes inside a row
    mask8 = mask.to(torch.uint8).to(DEV)
    kv_dev = torch.tensor(kv, dtype=torch.int32, device=DEV)
    out_pad = torch.empty(B * S, 2 * H * 64, device=DEV, dtype=torch.bfloat16)
    K().attn_prefill(q, kc, vc, B, S, H, mask8, kv_dev, causal, out_pad)
    pk = _pack(kv, B, S)
    gi = pk.gather[:pk.n_valid].long()
    kc_nan, vc_nan = kc.clone(), vc.clone()
    for b, k0 in enumerate(kv):
        kc_nan[b, :, :k0] = float("nan")
        vc_nan[b, :, :k0] = float("nan")
    q_pk = q.reshape(B * S, H * 64)[gi].contiguous()
    out_pk = torch.full((pk.n_valid + 5, 2 * H * 64), 3.0, device=DEV, dtype=torch.bfloat16)
    K().attn_prefill_packed(q_pk, kc_nan, vc_nan, B, S, H, mask8, kv_dev, pk.q_offset,
                            pk.n_valid, causal, out_pk)
    # the same launch writing the MFMA tile layout (the K6 prefill input) holds the same rows
    out_t = torch.full((K().split_numel(pk.n_valid, H * 64, True),), 3.0, device=DEV,
                       dtype=torch.bfloat16)
    K().attn_prefill_packed(q_pk, kc_nan, vc_nan, B, S, H, mask8, kv_dev, pk.q_offset,
                            pk.n_valid, causal, out_t, out_tiled=True)
    torch.cuda.synchronize()
    assert torch.equal(out_pk[:pk.n_valid], out_pad[gi])
    assert bool((out_pk[pk.n_valid:] == 3).all())
    assert torch.equal(K().untile_matrix(out_t, pk.n_valid, 2 * H * 64), out_pk[:pk.n_valid])


@pytest.mark.parametrize("packed", [False, True])
def test_attn_prefill_row_holes(packed):
    """row_holes[b] == 0 (the key mask of row b is the run [kv_start, S)) lets the kernel skip
    the mask: same outputs bit for bit as reading it.  The flag is a promise: set on the row
    that has holes, that row's holes are ignored and only its outputs change."""
    g = torch.Generator().manual_seed(77 + packed)
    B, H, S, slots = 6, 3, 300, 320
    q = bf(torch.randn(B, S, H, 64, generator=g) * 0.125).to(DEV)
    kc = bf(torch.randn(B, H, slots, 64, generator=g)).to(DEV)
    vc = bf(torch.randn(B, H, slots, 64, generator=g)).to(DEV)
    kv = [0, 299, 170, 300, 64, 1]
    mask = torch.ones(B, S, dtype=torch.bool)
    for b, k0 in enumerate(kv):
        mask[b, :k0] = False
    mask[4, 200:230] = False                       # the only row with holes
    mask8 = mask.to(torch.uint8).to(DEV)
    kv_dev = torch.tensor(kv, dtype=torch.int32, device=DEV)
    holes = torch.tensor([0, 0, 0, 0, 1, 0], dtype=torch.uint8, device=DEV)
    if packed:
        pk = _pack(kv, B, S)
        gi = pk.gather[:pk.n_valid].long()
        qq, rows = q.reshape(B * S, H * 64)[gi].contiguous(), pk.n_valid
        row_b = torch.repeat_interleave(torch.arange(B), torch.tensor([S - k for k in kv]))
    else:
        qq, rows = q, B * S
        row_b = torch.arange(B).repeat_interleave(S)

    def run(row_holes):
        out = torch.full((rows, 2 * H * 64), 3.0, device=DEV, dtype=torch.bfloat16)
        if packed:
            K().attn_prefill_packed(qq, kc, vc, B, S, H, mask8, kv_dev, pk.q_offset, rows, True,
                                    out, row_holes=row_holes)
        else:
            K().attn_prefill(qq, kc, vc, B, S, H, mask8, kv_dev, True, out, row_holes=row_holes)
        torch.cuda.synchronize()
        return out

    ref = run(None)
    assert torch.equal(run(holes), ref)
    wrong = run(torch.zeros_like(holes)).cpu()
    refc = ref.cpu()
    same = (wrong == refc).all(1)
    assert bool(same[row_b != 4].all())
    assert not bool(same[row_b == 4].all())


@pytest.mark.parametrize("packed", [False, True])
def test_attn_prefill_lead_exact(packed):
    """K4c: the first 64 queries at or after kv_start of each row come out as exact causal
    attention (fp64 reference from the same fp32 projection output: RMSNorm scale, 3D RoPE,
    softmax scale 1/8, key mask with holes) to fp32 rounding; every other output row keeps K4a's
    value bit for bit."""
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    g = torch.Generator().manual_seed(5 + packed)
    B, H, S, slots = 5, 3, 150, 160
    d = 64 * H
    cfg = _cfg(d, H)
    kv = [0, 40, 149, 150, 100]
    mask = torch.ones(B, S, dtype=torch.bool)
    for b, k0 in enumerate(kv):
        mask[b, :k0] = False
    mask[0, 3:6] = False                       # holes among the lead keys
    mask[4, 110:112] = False
    qkv = torch.randn(B * S, 3 * d, generator=g)
    rstd = 0.5 + torch.rand(B * S, generator=g)
    pos = torch.randint(0, 31, (B * S, 3), generator=g)
    rope = RotaryEmbedding3D(64, cfg.max_x, cfg.max_y, cfg.max_z)
    tab = rope.device_table(DEV)
    geom = (rope.max_x, rope.max_y, rope.max_z, rope.px, rope.py, rope.pz)
    kv_dev = torch.tensor(kv, dtype=torch.int32, device=DEV)
    mask8 = mask.to(torch.uint8).to(DEV)
    kc = torch.zeros(B, H, slots, 64, device=DEV, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    if packed:
        pk = _pack(kv, B, S)
        gi = pk.gather.long().cpu()
        rows = pk.n_tokens
        qkv_r, rstd_r, pos_r = qkv[gi], rstd[gi], pos[gi]
        q = torch.empty(rows, d, device=DEV, dtype=torch.bfloat16)
        K().qkv_rope_cache_packed(qkv_r.to(DEV), rstd_r.to(DEV), pos_r.to(DEV), tab, geom,
                                  pk.token_row, pk.token_slot, H, 0.125, q, kc, vc)
        out = torch.full((rows, 2 * d), 5.0, device=DEV, dtype=torch.bfloat16)
        K().attn_prefill_packed(q, kc, vc, B, S, H, mask8, kv_dev, pk.q_offset, pk.n_valid,
                                True, out)
        row_of = lambda b, i: int(pk.q_offset[b]) + i - kv[b]   # noqa: E731
    else:
        rows = B * S
        qkv_r, rstd_r, pos_r = qkv, rstd, pos
        q = torch.empty(rows, d, device=DEV, dtype=torch.bfloat16)
        K().qkv_rope_cache(qkv.to(DEV), rstd.to(DEV), pos.to(DEV), tab, geom, B, S, H, 0.125, q,
                           kc, vc)
        out = torch.empty(rows, 2 * d, device=DEV, dtype=torch.bfloat16)
        K().attn_prefill(q, kc, vc, B, S, H, mask8, kv_dev, True, out)
        row_of = lambda b, i: b * S + i                            # noqa: E731
    before = out.clone()
    K().attn_prefill_lead(qkv_r.to(DEV), rstd_r.to(DEV), pos_r.to(DEV), tab, geom, 0.125, B, S,
                          H, mask8, kv_dev, pk.q_offset if packed else None, rows, out)
    torch.cuda.synchronize()
    # fp64 reference over the padded batch
    y = (qkv.double() * rstd.double()[:, None]).view(B, S, 3, H, 64)
    tabs = rp.rope3d_tables(cfg)
    p3 = pos.view(B, S, 3)
    qr = rp.apply_rope3d(y[:, :, 0], p3, tabs, cfg).double()
    kr = rp.apply_rope3d(y[:, :, 1], p3, tabs, cfg).double()
    vis = mask.clone()
    for b, k0 in enumerate(kv):
        vis[b, :k0] = False
    ref = rp.attention(qr.transpose(1, 2), kr.transpose(1, 2), y[:, :, 2].transpose(1, 2), vis,
                       True).transpose(1, 2)                           # [B, S, H, 64]
    got = unsplit(out).view(rows, H, 64)
    lead = torch.zeros(rows, dtype=torch.bool)
    for b, k0 in enumerate(kv):
        for i in range(k0, min(k0 + 64, S)):
            r = row_of(b, i)
            lead[r] = True
            err = (got[r].double() - ref[b, i]).abs()
            assert bool((err <= 1e-5 + 1e-5 * ref[b, i].abs()).all()), (b, i, err.max().item())
    assert torch.equal(out[~lead.to(DEV)], before[~lead.to(DEV)])
    # the tile-layout output (the K6 prefill input) gets the same values in the same rows
    out_t = K().tile_matrix(before)
    K().attn_prefill_lead(qkv_r.to(DEV), rstd_r.to(DEV), pos_r.to(DEV), tab, geom, 0.125, B, S,
                          H, mask8, kv_dev, pk.q_offset if packed else None, rows, out_t,
                          out_tiled=True)
    assert torch.equal(K().untile_matrix(out_t, rows, 2 * d), out)


# ---------------------------------------------------------------------------- K4b decode

@pytest.mark.parametrize("split_len,slots,t", [(128, 700, 611), (256, 700, 611),
                                               (4096, 700, 611),       # 32-slot wave tiles
                                               (4096, 2600, 2511),     # 64-slot tiles, one split
                                               (2176, 5000, 4711)])    # 64-slot tiles, 3 splits
@pytest.mark.parametrize("with_mask", [True, False])
def test_attn_decode(split_len, slots, t, with_mask):
    g = torch.Generator().manual_seed(split_len + slots + with_mask)
    B, H, S = 5, 3, 300
    q = bf(torch.randn(B, H, 64, generator=g) * 0.125)
    kc = bf(torch.randn(B, H, slots, 64, generator=g))
    vc = bf(torch.randn(B, H, slots, 64, generator=g))
    pm = _masks(B, S, "left", g) if with_mask else None
    if with_mask:
        pm[2, :100] = False
        pm[2, 100:] = True
        pm[2, 250:260] = False                       # a hole inside the prompt
    kv_start = None
    if pm is not None:
        kv_start = torch.where(pm.any(1), pm.float().argmax(1), torch.full((B,), S))
        kv_start = kv_start.to(torch.int32).to(DEV)
    ws_n = K().attn_decode_workspace_bytes(B, H, slots, split_len) // 4
    ws = torch.empty(max(ws_n, 1), device=DEV) if ws_n else None
    out = torch.empty(B, 2 * H * 64, device=DEV, dtype=torch.bfloat16)
    holes = None
    if pm is not None:
        # rows without holes skip the mask; row 2 has one and must keep reading it
        holes = torch.tensor([0 if (not pm[b].any() or bool(pm[b, int(kv_start[b]):].all()))
                              else 1 for b in range(B)], dtype=torch.uint8)
        assert holes[2] == 1 and holes.sum() == 1
        holes = holes.to(DEV)
    order = torch.tensor([3, 0, 4, 2, 1], dtype=torch.int32, device=DEV)
    for dev_seq, use_holes, use_order in ((False, False, False), (True, False, True),
                                          (True, True, True)):
        seq_dev = torch.tensor([t], dtype=torch.int32, device=DEV) if dev_seq else None
        K().attn_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), B, H,
                        None if pm is None else pm.to(torch.uint8).to(DEV), S if pm is not None
                        else 0, kv_start, t, seq_dev, ws, split_len, out,
                        row_holes=holes if use_holes else None,
                        row_order=order if use_order else None)
        torch.cuda.synchronize()
        keymask = torch.ones(B, t + 1, dtype=torch.bool)
        if pm is not None:
            keymask[:, :S] = pm
        ref = rp.attention((q.double() * 8 / LOG2E)[:, :, None], kc[:, :, :t + 1].double(),
                           vc[:, :, :t + 1].double(), keymask, causal=False)[:, :, 0]
        # fp32 softmax and accumulation; the probabilities enter the PV product (and the row sum)
        # rounded to bf16, as in the prefill kernel: bf16-level agreement
        close_bf16(unsplit(out).view(B, H, 64), ref.float(), atol=4e-3, rtol=1e-2)


@pytest.mark.parametrize("split_len,slots,t", [(128, 900, 777), (384, 900, 777),
                                               (1024, 900, 777), (2176, 2600, 2477)])
def test_attn_decode_rope_equals_k2_then_decode(split_len, slots, t):
    """The fused decode launch writes the same K/V into slot t (to 1 bf16 ulp of the rotation's
    rounding) and returns the same attention as mdl_qkv_rope_cache + mdl_attn_decode (32- and
    64-slot wave tiles)."""
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    g = torch.Generator().manual_seed(split_len)
    B, H, S = 6, 3, 400
    d = 64 * H
    qkv = torch.randn(B, 3 * d, generator=g).to(DEV)
    rstd = (0.5 + torch.rand(B, generator=g)).to(DEV)
    pos = torch.randint(0, 35, (B, 3), generator=g).to(DEV)
    rope = RotaryEmbedding3D(64, 32, 32, 8)
    tab, geom = rope.device_table(DEV), (32, 32, 8, rope.px, rope.py, rope.pz)
    kc0 = bf(torch.randn(B, H, slots, 64, generator=g)).to(DEV)
    vc0 = bf(torch.randn(B, H, slots, 64, generator=g)).to(DEV)
    pm = _masks(B, S, "left", g)
    pm[1, 300:310] = False
    kv_start = torch.where(pm.any(1), pm.float().argmax(1), torch.full((B,), S))
    kv_start = kv_start.to(torch.int32).to(DEV)
    pm = pm.to(torch.uint8).to(DEV)
    seq_dev = torch.tensor([t], dtype=torch.int32, device=DEV)
    ws_n = K().attn_decode_workspace_bytes(B, H, slots, split_len) // 4
    ws = torch.empty(max(ws_n, 1), device=DEV) if ws_n else None
    order = torch.argsort(kv_start).to(torch.int32)
    # unfused reference path
    kc1, vc1 = kc0.clone(), vc0.clone()
    q = torch.empty(B, d, device=DEV, dtype=torch.bfloat16)
    out1 = torch.empty(B, 2 * d, device=DEV, dtype=torch.bfloat16)
    K().qkv_rope_cache(qkv, rstd, pos, tab, geom, B, 1, H, 0.125, q, kc1, vc1, slot_dev=seq_dev)
    K().attn_decode(q, kc1, vc1, B, H, pm, S, kv_start, 0, seq_dev, ws, split_len, out1,
                    row_order=order)
    # fused
    kc2, vc2 = kc0.clone(), vc0.clone()
    out2 = torch.empty_like(out1)
    K().attn_decode_rope(qkv, rstd, pos, tab, geom, 0.125, kc2, vc2, B, H, pm, S, kv_start, 0,
                         seq_dev, ws, split_len, out2, row_order=order)
    torch.cuda.synchronize()
    others = torch.ones(slots, dtype=torch.bool)
    others[t] = False
    assert torch.equal(kc1[:, :, others.to(DEV)], kc2[:, :, others.to(DEV)])
    assert torch.equal(vc1, vc2)
    close_bf16(kc2[:, :, t], kc1[:, :, t].float(), atol=1e-6, rtol=8e-3)
    assert torch.allclose(unsplit(out2), unsplit(out1), rtol=2e-3, atol=2e-4)


# ---------------------------------------------------------------------------- head + state

@pytest.mark.parametrize("d", [128, 768, 1280])
def test_lm_head_and_argmax(d):
    g = torch.Generator().manual_seed(d)
    M, V = 50, 14
    x = torch.randn(M, d, generator=g) * 3
    gamma = 1 + 0.1 * torch.randn(d, generator=g)
    w = torch.randn(V, d, generator=g) / math.sqrt(d)
    w[9] = w[4]                                        # exact tie between tokens 4 and 9
    rows = torch.randperm(M, generator=g)[:20].to(torch.int32)
    logits = torch.empty(20, V, device=DEV)
    tok = torch.empty(20, dtype=torch.int64, device=DEV)
    K().lm_head(x.to(DEV), rows.to(DEV), 20, gamma.to(DEV), 1e-5, w.to(DEV), logits, tok)
    torch.cuda.synchronize()
    ref = rp.rmsnorm(x[rows.long()].double(), gamma.double(), 1e-5) @ w.double().T
    assert torch.allclose(logits.cpu().double(), ref, atol=2e-5, rtol=1e-5)
    lg = logits.cpu()
    assert torch.equal(tok.cpu(), lg.argmax(-1))
    # forcing the tie to be the max: first index must win
    w2 = torch.zeros(V, d)
    w2[4] = w2[9] = 1.0
    t2 = torch.empty(20, dtype=torch.int64, device=DEV)
    K().lm_head(x.abs().to(DEV), rows.to(DEV), 20, torch.ones(d, device=DEV), 1e-5, w2.to(DEV),
                None, t2)
    torch.cuda.synchronize()
    assert bool((t2.cpu() == 4).all())


def test_grid_kernels_match_reference_golden():
    gs = np.load("tests/golden/grid_state.npz")
    toks = torch.from_numpy(gs["tokens"])
    n, steps = toks.shape
    gx = torch.from_numpy(gs["x0"]).to(torch.int32).to(DEV)
    gy = torch.from_numpy(gs["y0"]).to(torch.int32).to(DEV)
    io = torch.from_numpy(gs["io0"]).to(torch.uint8).to(DEV)
    pos = torch.empty(n, 3, dtype=torch.int64, device=DEV)
    counters = torch.tensor([5, 9], dtype=torch.int32, device=DEV)
    trace = []
    for s in range(steps):
        K().grid_step(toks[:, s].contiguous().to(DEV), gx, gy, io, pos, counters)
        trace.append(pos.cpu().numpy().copy())
    assert np.array_equal(np.stack(trace, 1), gs["positions"])
    fin = np.stack([gx.cpu().numpy(), gy.cpu().numpy(), io.cpu().numpy()], 1).astype(np.int64)
    assert np.array_equal(fin, gs["final"])
    assert counters.cpu().tolist() == [5 + steps, 9 + steps]
    B = gs["p_ids"].shape[0]
    ox, oy = torch.empty(B, dtype=torch.int32, device=DEV), torch.empty(B, dtype=torch.int32,
                                                                        device=DEV)
    oio = torch.empty(B, dtype=torch.uint8, device=DEV)
    kvs = torch.empty(B, dtype=torch.int32, device=DEV)
    last = torch.empty(B, dtype=torch.int32, device=DEV)
    mask = torch.from_numpy(gs["p_mask"])
    holes = torch.empty(B, dtype=torch.uint8, device=DEV)
    K().grid_init(torch.from_numpy(gs["p_ids"]).to(DEV), torch.from_numpy(gs["p_pos"]).to(DEV),
                  mask.to(torch.uint8).to(DEV), ox, oy, oio, kvs, last, row_holes=holes)
    init = np.stack([ox.cpu().numpy(), oy.cpu().numpy(), oio.cpu().numpy()], 1).astype(np.int64)
    assert np.array_equal(init, gs["init"])
    L = mask.shape[1]
    n_valid = mask.sum(1)
    first = torch.where(n_valid > 0, mask.float().argmax(1), torch.full((B,), L))
    assert torch.equal(kvs.cpu().long(), first)
    assert torch.equal(last.cpu().long(), torch.arange(B) * L + (n_valid - 1).clamp(min=0))
    # a row has holes iff its valid positions are not exactly [first, L)
    want = torch.tensor([0 if n_valid[b] == L - first[b] else 1 for b in range(B)],
                        dtype=torch.uint8)
    assert torch.equal(holes.cpu(), want)
    assert want.sum() > 0 and (want == 0).sum() > 0          # the fixture exercises both kinds


def test_grid_init_row_shift_equals_chunk_padding():
    """Rows left-padded together in one wide batch with row_shift = S - L_c give exactly the
    grid state and lengths-1 row that grid_init gives on each chunk padded to its own width L_c
    (including rows whose lengths-1 index falls in the padding)."""
    from mdlarc_scale_amd.inference import left_pad_batch

    rng = np.random.default_rng(11)
    chunk = 4
    prompts = []
    for i in range(11):
        n = int(rng.integers(1, 40))
        toks = [10] + [int(t) for t in rng.integers(0, 14, n)]      # START + random tokens
        prompts.append(toks)
    def run(ps, shift=None):
        ids, pos, mask = left_pad_batch(ps, DEV)
        B = len(ps)
        o = [torch.empty(B, dtype=torch.int32, device=DEV) for _ in range(2)]
        io = torch.empty(B, dtype=torch.uint8, device=DEV)
        last = torch.empty(B, dtype=torch.int32, device=DEV)
        K().grid_init(ids, pos, mask.to(torch.uint8), o[0], o[1], io, None, last,
                      row_shift=None if shift is None else shift.to(DEV))
        return o[0].cpu(), o[1].cpu(), io.cpu(), last.cpu(), ids.cpu(), ids.shape[1]
    gx, gy, io, last, ids, S = run(prompts)
    widths = [max(len(p) for p in prompts[c:c + chunk]) for c in range(0, len(prompts), chunk)]
    shift = torch.tensor([S - widths[i // chunk] for i in range(len(prompts))], dtype=torch.int32)
    sx, sy, sio, slast, _, _ = run(prompts, shift)
    hit_pad = 0
    for c0 in range(0, len(prompts), chunk):
        cx, cy, cio, clast, cids, L = run(prompts[c0:c0 + chunk])
        for j in range(cx.shape[0]):
            b = c0 + j
            assert (sx[b], sy[b], sio[b]) == (cx[j], cy[j], cio[j]), f"row {b}"
            lc = int(clast[j]) - j * L                       # index inside the chunk's padding
            assert int(slast[b]) - b * S == S - L + lc
            assert int(ids.view(-1)[slast[b]]) == int(cids.view(-1)[clast[j]])
            hit_pad += int(lc < L - len(prompts[b]))
    assert hit_pad > 0                                       # some index lands in the padding
    assert not torch.equal(slast, last)                      # the shift moved some rows


@pytest.mark.parametrize("d,with_ex", [(256, True), (768, True), (1280, False)])
def test_decode_embed_equals_grid_step_plus_embed(d, with_ex):
    """The fused decode-step entry equals mdl_grid_step followed by mdl_embed_rmsnorm."""
    g = torch.Generator().manual_seed(d)
    B, V, NE = 37, 14, 9
    tok = torch.randn(V, d, generator=g).to(torch.bfloat16).to(DEV)
    ex = torch.randn(NE, d, generator=g).to(torch.bfloat16).to(DEV)
    gamma = (1 + 0.1 * torch.randn(d, generator=g)).to(DEV)
    ex_ids = torch.randint(0, NE, (B,), generator=g).to(DEV) if with_ex else None
    state0 = (torch.randint(0, 33, (B,), generator=g).to(torch.int32),
              torch.randint(0, 31, (B,), generator=g).to(torch.int32),
              torch.randint(0, 2, (B,), generator=g).to(torch.uint8))
    outs = []
    for fused in (False, True):
        gx, gy, io = (s.clone().to(DEV) for s in state0)
        counters = torch.tensor([3, 7], dtype=torch.int32, device=DEV)
        pos = torch.empty(B, 3, dtype=torch.int64, device=DEV)
        x = torch.empty(B, d, device=DEV)
        xs = torch.empty(B, 2 * d, device=DEV, dtype=torch.bfloat16)
        r = torch.empty(B, device=DEV)
        for step in range(5):
            token = torch.randint(0, V, (B,), generator=torch.Generator().manual_seed(step)).to(DEV)
            if fused:
                K().decode_embed(token, ex_ids, tok, ex if with_ex else None, gamma, 1e-5, gx, gy,
                                 io, pos, counters, x, xs, r)
            else:
                K().grid_step(token, gx, gy, io, pos, counters)
                K().embed_rmsnorm(token, ex_ids, tok, ex if with_ex else None, 1, gamma, 1e-5, x,
                                  xs, r)
        torch.cuda.synchronize()
        outs.append([t.cpu() for t in (gx, gy, io, counters, pos, x, xs, r)])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert outs[1][3].tolist() == [8, 12]


@pytest.mark.parametrize("d,V", [(128, 14), (768, 14), (1280, 14), (256, 20)])
def test_decode_head_equals_lm_head_plus_commit(d, V):
    g = torch.Generator().manual_seed(d + V)
    B, cols = 45, 16
    x = (torch.randn(B, d, generator=g) * 2).to(DEV)
    gamma = (1 + 0.1 * torch.randn(d, generator=g)).to(DEV)
    w = (torch.randn(V, d, generator=g) / math.sqrt(d)).to(DEV)
    w[V - 1] = w[2]                                  # exact tie: first index must win
    ref_logits = torch.empty(B, V, device=DEV)
    ref_tok = torch.empty(B, dtype=torch.int64, device=DEV)
    K().lm_head(x, None, B, gamma, 1e-5, w, ref_logits, ref_tok)
    out_ref = torch.full((B, cols), -1, dtype=torch.int64, device=DEV)
    fin_ref = torch.full((B,), -1, dtype=torch.int32, device=DEV)
    counters = torch.tensor([0, 9], dtype=torch.int32, device=DEV)
    K().decode_commit(ref_tok, out_ref, 0, counters, fin_ref, 4, 2)
    logits = torch.empty(B, V, device=DEV)
    tok = torch.empty(B, dtype=torch.int64, device=DEV)
    out = torch.full((B, cols), -1, dtype=torch.int64, device=DEV)
    fin = torch.full((B,), -1, dtype=torch.int32, device=DEV)
    K().decode_head(x, gamma, 1e-5, w, logits, tok, out, 0, counters, fin, 4, 2)
    torch.cuda.synchronize()
    assert torch.equal(tok.cpu(), ref_tok.cpu())
    assert torch.equal(out.cpu(), out_ref.cpu()) and torch.equal(fin.cpu(), fin_ref.cpu())
    assert (fin.cpu() == 5).sum() == (tok.cpu() == 2).sum()      # token 2 stands for END here
    ref = rp.rmsnorm(x.cpu().double(), gamma.cpu().double(), 1e-5) @ w.cpu().double().T
    assert torch.allclose(logits.cpu().double(), ref, atol=2e-5, rtol=1e-5)
    assert not bool((tok.cpu() == V - 1).any())      # the tied duplicate of slot 2 never wins


def test_head_constraints_equal_oracle_rule():
    """The head kernels with fused logit constraints return the plain kernel's logits after the
    oracle's restatement of _apply_logit_constraints (src/inference.py:285-364), which the
    reference's own outputs pin bit for bit (tests/golden/constraints.npz): the same fp32
    subtractions in the same order, so bit-identical logits and argmax.  The rows cover every
    branch: palette on / off, target shape on / off (-1), x below / at / past the width, y
    below / past the height, and the disallowed START / IO_SEP (which would otherwise win: their
    weight rows are scaled up); the penalties are those of the reference fixture's cases."""
    from tests.golden_io import constraint_cases

    g = torch.Generator().manual_seed(4)
    B, d, V = 64, 256, 14
    x = torch.randn(B, d, generator=g).to(DEV)
    gamma = (1 + 0.1 * torch.randn(d, generator=g)).to(DEV)
    w = torch.randn(V, d, generator=g) / math.sqrt(d)
    w[10] *= 3
    w[12] *= 3
    w = w.to(DEV)
    plain = torch.empty(B, V, device=DEV)
    K().lm_head(x, None, B, gamma, 1e-5, w, plain, None)
    pens = sorted({(c["palette_penalty"], c["shape_penalty"]) for c in constraint_cases()})
    assert len(pens) >= 3
    for pp, sp in pens:
        pal = torch.rand(B, 10, generator=g) < 0.5
        pal[::5] = True                                       # rows without palette penalty
        shape = torch.randint(1, 6, (B, 2), generator=g)
        shape[::4] = -1                                       # rows without target shape
        shape[1::8, 0] = -1                                   # h < 0 alone: no shape either
        gx = torch.randint(0, 7, (B,), generator=g).to(torch.int32)
        gy = torch.randint(0, 7, (B,), generator=g).to(torch.int32)
        gx[2], gy[2] = shape[2, 1], shape[2, 0]               # exactly at the width / height
        hc = K().HeadConstraints((10, 12), pal.to(DEV), pp, shape.to(DEV), gx.to(DEV),
                                 gy.to(DEV), sp)
        ref = rp.apply_logit_constraints(
            plain.cpu().clone(), gx.long(), gy.long(),
            rp.OracleConstraints(palette_mask=pal, target_shape=shape, palette_penalty=pp,
                                 shape_penalty=sp, disallow_tokens=(10, 12)))
        got = torch.empty(B, V, device=DEV)
        tok = torch.empty(B, dtype=torch.int64, device=DEV)
        K().lm_head(x, None, B, gamma, 1e-5, w, got, tok, hc)
        out = torch.full((B, 4), -1, dtype=torch.int64, device=DEV)
        dlog = torch.empty(B, V, device=DEV)
        dtok = torch.empty(B, dtype=torch.int64, device=DEV)
        K().decode_head(x, gamma, 1e-5, w, dlog, dtok, out, 1, None, None, 0, 13, hc)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), ref), (pp, sp)
        assert torch.equal(dlog.cpu(), ref), (pp, sp)
        assert torch.equal(tok.cpu(), ref.argmax(-1)) and torch.equal(dtok.cpu(), tok.cpu())
        assert torch.equal(out[:, 1].cpu(), tok.cpu())
        assert not bool(((tok == 10) | (tok == 12)).any())
        assert not torch.equal(plain.argmax(-1).cpu(), tok.cpu())  # the constraints changed tokens
        has = (shape[:, 0] >= 0) & (shape[:, 1] >= 0)
        for cond in (has & (gx >= shape[:, 1]), has & (gx < shape[:, 1]),
                     has & (gy >= shape[:, 0]), has & (gy < shape[:, 0]), ~has):
            assert bool(cond.any())                           # every branch is exercised


def test_build_prompts_equals_host_tokeniser():
    """mdl_build_prompts (dihedral transform, colour permutation, tokens, 3D positions, left
    padding on the device) equals the host path -- the data-format functions pinned by the
    reference's own known-answer tests -- exactly, on random tasks: 0-3 demonstration pairs,
    grids from 1x1 to 30x30, all 8 transforms x 3 colour permutations."""
    from mdlarc_scale_amd import inference as inf

    rng = np.random.default_rng(21)

    def grid(h=None, w=None):
        h = int(rng.integers(1, 31)) if h is None else h
        w = int(rng.integers(1, 31)) if w is None else w
        g = rng.integers(1, 10, size=(h, w))
        g[rng.random((h, w)) < 0.5] = 0
        return g.tolist()

    for trial in range(7):
        n_pairs = trial % 4
        pairs = [{"input": grid(), "output": grid()} for _ in range(n_pairs)]
        test_in = grid(1, 1) if trial == 5 else (grid(30, 30) if trial == 6 else grid())
        task = {"train": pairs, "test": [{"input": test_in}]}
        variants = inf._build_variants(task, 0, True, 3, 1, False, None, None)
        ids_h, pos_h, mask_h = inf.left_pad_batch([v.tokens for v in variants], DEV)
        grids = inf._task_grids(task, 0, True)
        ids_d, pos_d, mask_d, lens = inf._device_prompts(grids, variants, 3, DEV)
        torch.cuda.synchronize()
        assert lens == [len(v.tokens) for v in variants]
        assert torch.equal(ids_d.cpu(), ids_h.cpu()), f"trial {trial}: tokens"
        assert torch.equal(pos_d.cpu(), pos_h.cpu()), f"trial {trial}: positions"
        assert torch.equal(mask_d.cpu(), mask_h.cpu()), f"trial {trial}: mask"


def test_decode_commit():
    B, cols = 6, 10
    out = torch.full((B, cols), -7, dtype=torch.int64, device=DEV)
    fin = torch.tensor([-1, -1, 3, -1, -1, -1], dtype=torch.int32, device=DEV)
    tok = torch.tensor([13, 2, 13, 11, 13, 0], dtype=torch.int64, device=DEV)
    K().decode_commit(tok, out, 6, None, fin, 4, 13)
    counters = torch.tensor([0, 8], dtype=torch.int32, device=DEV)
    K().decode_commit(tok.flip(0).contiguous(), out, 0, counters, fin, 4, 13)
    torch.cuda.synchronize()
    assert out[:, 6].cpu().tolist() == [13, 2, 13, 11, 13, 0]
    assert out[:, 8].cpu().tolist() == [0, 13, 11, 13, 2, 13]
    assert fin.cpu().tolist() == [2, 4, 3, 4, 2, 4]


def test_capi_rejects_bad_arguments_before_launch():
    from mdlarc_scale_amd import _lib

    L = _lib.lib()
    x = torch.zeros(16, 64, device=DEV)
    # head_dim must be 64
    assert L.mdl_attn_prefill(x.data_ptr(), x.data_ptr(), x.data_ptr(), 1, 4, 1, 32, 4, None,
                              None, None, 1, x.data_ptr(), 0, None) == -4
    # cache overflow: slot0 + seq > slots
    assert L.mdl_qkv_rope_cache(x.data_ptr(), 192, None, x.data_ptr(), x.data_ptr(), 1, 4, 1, 64,
                                32, 32, 8, 10, 10, 12, 0.125, x.data_ptr(), x.data_ptr(),
                                x.data_ptr(), 1, 4, 1, None, None) == -5
    # misaligned pointer
    assert L.mdl_swiglu(x.data_ptr() + 2, 16, None, None, None, 1, 8, x.data_ptr(), 0,
                        None) == -2
    # workspace too small for a multi-split decode
    assert L.mdl_attn_decode(x.data_ptr(), x.data_ptr(), x.data_ptr(), 1, 1, 64, 1024, None, 0,
                             None, None, None, 5, None, None, 0, 128, x.data_ptr(), 0,
                             None) == -6
    with pytest.raises(RuntimeError, match="head_dim"):
        _lib.check(-4, "probe")


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k", [(256, 2304, 768), (256, 768, 2048), (128, 5504, 1024),
                                   (64, 1280, 3392), (3, 80, 64), (17, 1408, 704),
                                   (100, 256, 96), (1000, 768, 256), (777, 2304, 768)])
def test_gemm_split(m, n, k):
    """K5, every compiled block shape and the automatic choice, against an fp64 CPU product of
    the same bf16 operands: (hi + lo) @ w^T to fp32 accumulation error (bound: 1e-5 of the sum
    of |products|, a few ulps per term at these K), rows and columns past the tiles included.
    For one block shape the four operand layouts (row-major / MFMA tiles, each operand) give
    identical bits, and so do two calls; the row-major weight may be the left half of the
    [W | W] prefill operand; the hipBLASLt [W | W] GEMM of the prefill agrees to the bound."""
    from mdlarc_scale_amd.engine import gemm_f32

    g = torch.Generator().manual_seed(m * 7 + n + k)
    x = torch.randn(m, k, generator=g) * 2.0
    hi = x.to(torch.bfloat16)
    lo = (x - hi.float()).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16)
    ref = (hi.double() + lo.double()) @ w.double().T
    bound = 1e-5 * ((hi.double().abs() + lo.double().abs()) @ w.double().abs().T) + 1e-30
    a = torch.cat([hi, lo], 1).to(DEV)
    w2 = torch.cat([w, w], 1).to(DEV)
    wd = w.to(DEV)
    at, wt = K().tile_matrix(a), K().tile_matrix(wd)

    def run(tile, a_op, a_tiled, w_op, w_tiled):
        out = torch.full((m, n), float("nan"), device=DEV)
        K().gemm_split(a_op, w_op, out, k, a_tiled=a_tiled, w_tiled=w_tiled, tile=tile)
        return out

    for t in list(range(1, K().gemm_split_tiles() + 1)) + [0]:
        out = run(t, at, True, wt, True)
        torch.cuda.synchronize()
        err = (out.cpu().double() - ref).abs()
        assert bool((err <= bound).all()), f"tile {t}: max err {err.max().item():.3e}"
        for a_op, a_t, w_op, w_t in ((at, True, wt, True), (a, False, w2, False),
                                     (a, False, wd, False), (at, True, w2, False),
                                     (a, False, wt, True)):
            assert torch.equal(run(t, a_op, a_t, w_op, w_t), out), f"tile {t} layouts"
    blas = torch.empty(m, n, device=DEV)
    gemm_f32(a, w2, blas)
    assert bool(((blas.cpu().double() - ref).abs() <= bound).all())


def test_tile_matrix_layout():
    """mdl_tile_matrix against the layout's definition: element (r, c) of a [rows, cols] matrix
    sits at 512 (r/16 * cols/32 + c/32) + 8 (16 ((c/8) % 4) + r % 16) + c % 8; padding rows 0."""
    rows, cols = 37, 96
    src = torch.arange(rows * cols, dtype=torch.float32).view(rows, cols)
    src_b = (src % 251).to(torch.bfloat16)
    got = K().tile_matrix(src_b.to(DEV)).cpu()
    r = torch.arange(48).view(48, 1).expand(48, cols)
    c = torch.arange(cols).view(1, cols).expand(48, cols)
    off = 512 * ((r // 16) * (cols // 32) + c // 32) + 8 * (16 * ((c // 8) % 4) + r % 16) + c % 8
    want = torch.zeros(48, cols, dtype=torch.bfloat16)
    want[:rows] = src_b
    assert got.numel() == 48 * cols
    assert torch.equal(got[off.reshape(-1)].view(48, cols), want)


@pytest.mark.parametrize("d", [256, 768, 800])
def test_producers_write_the_tile_layout(d):
    """Every producer of a decode GEMM input writes, with the tile layout selected, exactly
    mdl_tile_matrix of its row-major output (padding rows left untouched).  d = 256 is one
    256-channel chunk per row, 768 three, 800 three and a tail (chunks after the first and the
    tail are addressed from the first chunk's offsets)."""
    g = torch.Generator().manual_seed(11 + d)
    B, F, H = 37, 704, 4

    def both(fn, numel_rows, cols):
        outs = []
        for tiled in (False, True):
            buf = torch.zeros((K().tile_rows(numel_rows) if tiled else numel_rows) * cols,
                              device=DEV, dtype=torch.bfloat16)
            fn(buf, tiled)
            outs.append(buf)
        torch.cuda.synchronize()
        assert torch.equal(K().tile_matrix(outs[0].view(numel_rows, cols)), outs[1])

    tok = torch.randn(14, d, generator=g).to(DEV)
    ex = torch.randn(5, d, generator=g).to(DEV)
    gamma = (1 + 0.1 * torch.randn(d, generator=g)).to(DEV)
    ids = torch.randint(0, 14, (B,), generator=g).to(DEV)
    exi = torch.randint(0, 5, (B,), generator=g).to(DEV)
    r = torch.empty(B, device=DEV)
    state = (torch.randint(0, 30, (B,), generator=g).to(torch.int32),
             torch.randint(0, 29, (B,), generator=g).to(torch.int32),
             torch.randint(0, 2, (B,), generator=g).to(torch.uint8))
    pos = torch.empty(B, 3, dtype=torch.int64, device=DEV)
    # the embedding entries write x (fp32 tile layout) and xs (bf16 tile layout) when tiled
    for embed in (lambda xb, xsb, t: K().embed_rmsnorm(ids, exi, tok, ex, 1, gamma, 1e-5, xb,
                                                       xsb, r, tiled=t),
                  lambda xb, xsb, t: K().decode_embed(ids, exi, tok, ex, gamma, 1e-5,
                                                      *(s.clone().to(DEV) for s in state), pos,
                                                      None, xb, xsb, r, tiled=t)):
        xr = torch.zeros(B, d, device=DEV)
        xsr = torch.zeros(B * 2 * d, device=DEV, dtype=torch.bfloat16)
        embed(xr, xsr, False)
        xt = torch.zeros(K().tile_rows(B) * d, device=DEV)
        xst = torch.zeros(K().tile_rows(B) * 2 * d, device=DEV, dtype=torch.bfloat16)
        embed(xt, xst, True)
        xt_only = torch.zeros_like(xt)
        embed(xt_only, None, True)                   # xs optional
        torch.cuda.synchronize()
        assert torch.equal(K().tile_f32(xr), xt)
        assert torch.equal(xt_only, xt)
        assert torch.equal(K().tile_matrix(xsr.view(B, 2 * d)), xst)
    x0 = torch.randn(B, d, generator=g).to(DEV)
    delta = torch.randn(B, d, generator=g).to(DEV)
    both(lambda buf, t: K().add_rmsnorm(x0.clone(), delta, None, gamma, 1e-5, buf, r, tiled=t),
         B, 2 * d)
    gu = torch.randn(B, 2 * F, generator=g).to(DEV)
    both(lambda buf, t: K().swiglu(gu, r, None, None, buf, tiled=t), B, 2 * F)
    if d != 256:
        return
    # decode attention, unfused and fused with K2, single split and split-K (combine kernel)
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D
    rope = RotaryEmbedding3D(64, 32, 32, 8)
    tab, geom = rope.device_table(DEV), (32, 32, 8, rope.px, rope.py, rope.pz)
    slots, t_pos = 300, 250
    kc = bf(torch.randn(B, H, slots, 64, generator=g)).to(DEV)
    vc = bf(torch.randn(B, H, slots, 64, generator=g)).to(DEV)
    q = bf(torch.randn(B, H * 64, generator=g) / 8).to(DEV)
    qkv = torch.randn(B, 3 * H * 64, generator=g).to(DEV)
    rstd = (0.5 + torch.rand(B, generator=g)).to(DEV)
    posr = torch.randint(0, 30, (B, 3), generator=g).to(DEV)
    for split_len in (128, 384):
        ws_n = K().attn_decode_workspace_bytes(B, H, slots, split_len) // 4
        ws = torch.empty(max(ws_n, 1), device=DEV)
        both(lambda buf, t: K().attn_decode(q, kc, vc, B, H, None, 0, None, t_pos, None, ws,
                                            split_len, buf, tiled=t), B, 2 * H * 64)
        both(lambda buf, t: K().attn_decode_rope(qkv, rstd, posr, tab, geom, 0.125, kc.clone(),
                                                 vc.clone(), B, H, None, 0, None, t_pos, None,
                                                 ws, split_len, buf, tiled=t), B, 2 * H * 64)


def test_add_rmsnorm_tiled_xs_half_block_width():
    """mdl_add_rmsnorm's tiled split output at d = 784 (d = 16 mod 32): the lo half of a row
    starts in the middle of a 32-column tile block, so its offsets are not the hi half's shifted
    by whole blocks; exactly mdl_tile_matrix of the row-major output."""
    g = torch.Generator().manual_seed(784)
    B, d = 37, 784
    gamma = (1 + 0.1 * torch.randn(d, generator=g)).to(DEV)
    x0 = torch.randn(B, d, generator=g).to(DEV)
    delta = torch.randn(B, d, generator=g).to(DEV)
    r = torch.empty(B, device=DEV)
    outs = []
    for tiled in (False, True):
        rows = K().tile_rows(B) if tiled else B
        buf = torch.zeros(rows * 2 * d, device=DEV, dtype=torch.bfloat16)
        x = x0.clone()
        K().add_rmsnorm(x, delta, None, gamma, 1e-5, buf, r, tiled=tiled)
        outs.append(buf)
    torch.cuda.synchronize()
    assert torch.equal(K().tile_matrix(outs[0].view(B, 2 * d)), outs[1])


@pytest.mark.parametrize("m,f,k", [(256, 2048, 768), (37, 704, 256), (64, 3392, 1280)])
def test_gemm_split_swiglu_equals_gemm_then_swiglu(m, f, k):
    """K5 with the SwiGLU epilogue (gate / up weights with 16-row blocks interleaved) writes the
    same split h, bit for bit, as K5 on [W_gate; W_up] followed by K3 (mdl_swiglu), for every
    block shape and the automatic choice, with and without rstd and biases."""
    g = torch.Generator().manual_seed(m + f + k)
    x = torch.randn(m, k, generator=g) * 2.0
    hi = x.to(torch.bfloat16)
    lo = (x - hi.float()).to(torch.bfloat16)
    at = K().tile_matrix(torch.cat([hi, lo], 1).to(DEV))
    wg = (torch.randn(f, k, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(f, k, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    w_il = K().tile_matrix(K().interleave_gate_up(wg, wu))
    w_cat = K().tile_matrix(torch.cat([wg, wu], 0))
    rstd = (0.5 + torch.rand(m, generator=g)).to(DEV)
    bg = (0.1 * torch.randn(f, generator=g)).to(DEV)
    bu = (0.1 * torch.randn(f, generator=g)).to(DEV)
    for t in list(range(1, K().gemm_split_tiles() + 1)) + [0]:
        for r, b1, b2 in ((rstd, bg, bu), (None, None, None)):
            fused = torch.zeros(K().split_numel(m, f, True), device=DEV, dtype=torch.bfloat16)
            K().gemm_split_swiglu(at, w_il, r, b1, b2, fused, m, f, k, tile=t)
            gu = torch.empty(m, 2 * f, device=DEV)
            K().gemm_split(at, w_cat, gu, k, a_tiled=True, w_tiled=True, tile=t)
            ref = torch.zeros_like(fused)
            K().swiglu(gu, r, b1, b2, ref, tiled=True)
            torch.cuda.synchronize()
            assert torch.equal(fused, ref), f"tile {t}"



@pytest.mark.parametrize("m,n,k", [(256, 2304, 768), (37, 768, 256), (64, 3840, 1280)])
def test_gemm_norm_equals_add_rmsnorm_then_gemm(m, n, k):
    """K5 with the RMSNorm prologue (x in the fp32 tile layout) gives the same bits as
    mdl_add_rmsnorm (xs tiled) followed by K5 for every block shape, and the same rstd to fp32
    rounding (the sum of squares is taken in another order); the head kernels read the tiled x
    as they read the row-major one."""
    g = torch.Generator().manual_seed(m + n + k)
    x = (torch.randn(m, k, generator=g) * 1.5).to(DEV)
    gamma = (1 + 0.1 * torch.randn(k, generator=g)).to(DEV)
    w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    wt = K().tile_matrix(w)
    xs = torch.zeros(K().split_numel(m, k, True), device=DEV, dtype=torch.bfloat16)
    rstd_ref = torch.empty(m, device=DEV)
    K().add_rmsnorm(x.clone(), None, None, gamma, 1e-5, xs, rstd_ref, tiled=True)
    xt = K().tile_f32(x)
    for t in list(range(1, K().gemm_split_tiles() + 1)) + [0]:
        ref = torch.empty(m, n, device=DEV)
        K().gemm_split(xs, wt, ref, k, a_tiled=True, w_tiled=True, tile=t)
        out = torch.full((m, n), float("nan"), device=DEV)
        rstd = torch.full((m,), float("nan"), device=DEV)
        K().gemm_norm(xt, gamma, 1e-5, wt, out, rstd, k, tile=t)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"tile {t}"
        assert torch.allclose(rstd, rstd_ref, rtol=2e-6, atol=0), f"tile {t}"
    # the head kernels on the tiled x
    V = 14
    wh = (torch.randn(V, k, generator=g) / math.sqrt(k)).to(DEV)
    lr, lt = torch.empty(m, V, device=DEV), torch.empty(m, V, device=DEV)
    K().lm_head(x, None, m, gamma, 1e-5, wh, lr, None)
    K().lm_head(xt.view(-1, k), None, m, gamma, 1e-5, wh, lt, None, x_tiled=True)
    torch.cuda.synchronize()
    assert torch.equal(lr, lt)


@pytest.mark.parametrize("m,h", [(256, 12), (37, 4), (64, 20)])
def test_gemm_norm_qkv_equals_gemm_norm_then_k2(m, h):
    """The decode qkv projection with K2 in its epilogue writes exactly what the store form
    followed by qkv_rope_cache (one token per row, slot from the device counter) writes: q, the
    slot-t K / V, rstd -- for every block shape; no other cache slot changes."""
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    g = torch.Generator().manual_seed(m + h)
    d, slots, t = 64 * h, 40, 29
    x = (torch.randn(m, d, generator=g) * 1.5).to(DEV)
    gamma = (1 + 0.1 * torch.randn(d, generator=g)).to(DEV)
    wt = K().tile_matrix((torch.randn(3 * d, d, generator=g) * 0.05).to(torch.bfloat16).to(DEV))
    pos = torch.randint(0, 35, (m, 3), generator=g).to(DEV)
    rope = RotaryEmbedding3D(64, 30, 30, 8)
    tab, geom = rope.device_table(DEV), (30, 30, 8, rope.px, rope.py, rope.pz)
    slot = torch.tensor([t], dtype=torch.int32, device=DEV)
    xt = K().tile_f32(x)
    cache0 = bf(torch.randn(m, h, slots, 64, generator=g)).to(DEV)
    for tl in list(range(1, K().gemm_split_tiles() + 1)) + [0]:
        qkv = torch.empty(m, 3 * d, device=DEV)
        rs1 = torch.empty(m, device=DEV)
        K().gemm_norm(xt, gamma, 1e-5, wt, qkv, rs1, d, tile=tl)
        q1 = torch.empty(m, d, device=DEV, dtype=torch.bfloat16)
        kc1, vc1 = cache0.clone(), cache0.clone()
        K().qkv_rope_cache(qkv, rs1, pos, tab, geom, m, 1, h, 0.125, q1, kc1, vc1, slot_dev=slot)
        q2 = torch.empty(m, d, device=DEV, dtype=torch.bfloat16)
        kc2, vc2 = cache0.clone(), cache0.clone()
        rs2 = torch.empty(m, device=DEV)
        K().gemm_norm_qkv(xt, gamma, 1e-5, wt, m, h, rs2, pos, tab, geom, 0.125, q2, kc2, vc2,
                          slot_dev=slot, tile=tl)
        torch.cuda.synchronize()
        assert torch.equal(q1, q2), f"tile {tl}"
        assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), f"tile {tl}"
        assert torch.equal(rs1, rs2), f"tile {tl}"
        others = torch.ones(slots, dtype=torch.bool)
        others[t] = False
        assert torch.equal(kc2[:, :, others.to(DEV)], cache0[:, :, others.to(DEV)])


@pytest.mark.parametrize("m,f,k", [(256, 2048, 768), (37, 704, 256), (64, 3392, 1280)])
def test_gemm_norm_swiglu_equals_unfused(m, f, k):
    """The gate / up projection with the RMSNorm prologue and the SwiGLU epilogue against
    mdl_add_rmsnorm + K5 + K3.  The fused rstd may differ from mdl_add_rmsnorm's in its last bit,
    which can move the lo half of a split value by one ulp (hi + lo holds h to 2^-17 relative):
    bound 3e-5 relative.  A missing rstd, bias or a wrong channel pairing is off by 1e-1."""
    g = torch.Generator().manual_seed(m + f + k + 1)
    x = (torch.randn(m, k, generator=g) * 1.5).to(DEV)
    gamma = (1 + 0.1 * torch.randn(k, generator=g)).to(DEV)
    wg = (torch.randn(f, k, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(f, k, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    bg = (0.1 * torch.randn(f, generator=g)).to(DEV)
    bu = (0.1 * torch.randn(f, generator=g)).to(DEV)
    w_il = K().tile_matrix(K().interleave_gate_up(wg, wu))
    xs = torch.zeros(K().split_numel(m, k, True), device=DEV, dtype=torch.bfloat16)
    rstd = torch.empty(m, device=DEV)
    K().add_rmsnorm(x.clone(), None, None, gamma, 1e-5, xs, rstd, tiled=True)
    xt = K().tile_f32(x)

    def unsplit_tiled(h):
        hb = h.view(-1)
        r = torch.arange(K().tile_rows(m), device=DEV).view(-1, 1)
        c = torch.arange(2 * f, device=DEV).view(1, -1)
        off = (512 * ((r // 16) * (2 * f // 32) + c // 32) + 8 * (16 * ((c // 8) % 4) + r % 16)
               + c % 8)
        full = hb[off]
        return full[:m, :f].float() + full[:m, f:].float()

    for t in list(range(1, K().gemm_split_tiles() + 1)) + [0]:
        ref = torch.zeros(K().split_numel(m, f, True), device=DEV, dtype=torch.bfloat16)
        K().gemm_split_swiglu(xs, w_il, rstd, bg, bu, ref, m, f, k, tile=t)
        got = torch.zeros_like(ref)
        K().gemm_norm_swiglu(xt, gamma, 1e-5, w_il, bg, bu, got, m, f, k, tile=t)
        torch.cuda.synchronize()
        a, b = unsplit_tiled(got), unsplit_tiled(ref)
        assert torch.allclose(a, b, rtol=3e-5, atol=1e-6), f"tile {t}"


@pytest.mark.parametrize("m,n,k", [(256, 768, 768), (37, 256, 704), (64, 1280, 3392)])
def test_gemm_split_residual(m, n, k):
    """K5 with the residual epilogue: x (fp32 tile layout) += (hi + lo) @ W^T (+ bias) gives
    exactly (x + K5's output) + bias, in place, for every block shape; rows past m untouched."""
    g = torch.Generator().manual_seed(m + n + k + 2)
    a = torch.randn(m, k, generator=g)
    hi = a.to(torch.bfloat16)
    lo = (a - hi.float()).to(torch.bfloat16)
    at = K().tile_matrix(torch.cat([hi, lo], 1).to(DEV))
    w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    wt = K().tile_matrix(w)
    x = torch.randn(m, n, generator=g).to(DEV)
    bias = (0.1 * torch.randn(n, generator=g)).to(DEV)
    for t in list(range(1, K().gemm_split_tiles() + 1)) + [0]:
        for b in (bias, None):
            out = torch.empty(m, n, device=DEV)
            K().gemm_split(at, wt, out, k, a_tiled=True, w_tiled=True, tile=t)
            want = x + out
            if b is not None:
                want = want + b
            xt = K().tile_f32(x)
            pad = xt.clone()
            K().gemm_split_residual(at, wt, xt, b, m, n, k, tile=t)
            torch.cuda.synchronize()
            assert torch.equal(K().untile_f32(xt, m, n), want), f"tile {t}"
            # padding rows of the last row block stay as they were
            full = K().untile_f32(xt, K().tile_rows(m), n)
            assert torch.equal(full[m:], K().untile_f32(pad, K().tile_rows(m), n)[m:])
