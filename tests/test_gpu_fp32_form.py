"""Kernel-level parity of the fp32 form on the GPU (a model whose parameters are fp32 keeps fp32
weights, an fp32 cache and fp32 attention, as the reference does: src/inference.py:522, :544),
called through the C ABI (mdlarc_scale_amd.kernels):

* K5 with the low weight part (mdl_gemm_norm / _swiglu / mdl_gemm_split_residual, w_lo): the
  product against an fp32 weight W to ~2^-16 relative of sum |a||W| (fp64 reference), while the
  same launch without w_lo (W rounded to bf16) is off by ~2^-9 and fails that bound;
* K2 with fp32 outputs (mdl_qkv_rope_cache(_packed), MDL_DTYPE_F32): q / K / V against the
  oracle's RMSNorm scale + 3D RoPE in fp64 to fp32 rounding;
* K4f (mdl_attn_prefill_f32, mdl_attn_decode_f32): attention over an fp32 cache against the
  oracle's SDPA in fp64 to ~1e-5 (a bf16 rounding of q, K or V would be ~1e-2 off).
"""

import pytest
import torch

from mdlarc_scale_amd.transformer import LOG2E
from oracle import reference_path as rp

pytestmark = pytest.mark.gpu

DEV = "cuda"


def K():
    from mdlarc_scale_amd import kernels

    return kernels


def unsplit(t):
    t = t.float().cpu()
    k = t.shape[-1] // 2
    return t[..., :k] + t[..., k:]


def untile_split(h, m, f):
    """hi + lo of a tiled split [tile_rows(m), 2f] bf16 buffer -> [m, f] fp32."""
    full = K().untile_matrix(h, K().tile_rows(m), 2 * f).float().cpu()
    return full[:m, :f] + full[:m, f:]


def lo_part(w):
    return (w - w.to(torch.bfloat16).float()).to(torch.bfloat16)


def _tiles():
    return list(range(1, K().gemm_split_tiles() + 1)) + [0]


def _close(got, ref, scale, rel, what):
    err = (got.double() - ref).abs()
    bound = rel * scale + 1e-7
    ratio = (err / bound).max().item()
    assert ratio <= 1.0, f"{what}: max err {err.max().item():.3e}, worst ratio {ratio:.2f}"
    return ratio


# ------------------------------------------------------------------------------ K5 with w_lo

@pytest.mark.parametrize("m,n,k", [(37, 768, 256), (600, 768, 256), (64, 3840, 1280)])
def test_gemm_norm_fp32_weight(m, n, k):
    """out = split(x * gamma) @ W^T with W fp32, every block shape, rstd as the plain form."""
    g = torch.Generator().manual_seed(m + n + k)
    x = torch.randn(m, k, generator=g) * 1.5
    gamma = 1 + 0.1 * torch.randn(k, generator=g)
    w = torch.randn(n, k, generator=g) * 0.05
    xd, gd = x.to(DEV), gamma.to(DEV)
    wt = K().tile_matrix(w.to(torch.bfloat16).to(DEV))
    wl = K().tile_matrix(lo_part(w).to(DEV))
    a = (x.double() * gamma.double())
    ref = a @ w.double().T
    scale = a.abs() @ w.double().abs().T
    xt = K().tile_f32(xd)
    for t in _tiles():
        out = torch.full((m, n), float("nan"), device=DEV)
        rstd = torch.empty(m, device=DEV)
        K().gemm_norm(xt, gd, 1e-5, wt, out, rstd, k, tile=t, w_lo=wl)
        torch.cuda.synchronize()
        _close(out.cpu(), ref, scale, 2 ** -15, f"tile {t}")
        want = 1 / torch.sqrt((x.double() ** 2).mean(1) + 1e-5)
        assert torch.allclose(rstd.cpu().double(), want, rtol=1e-5)
    # without the low part the weight is bf16: the same bound fails (the test resolves it)
    out = torch.empty(m, n, device=DEV)
    K().gemm_norm(xt, gd, 1e-5, wt, out, None, k)
    torch.cuda.synchronize()
    with pytest.raises(AssertionError):
        _close(out.cpu(), ref, scale, 2 ** -15, "bf16 weight")


@pytest.mark.parametrize("m,f,k", [(37, 704, 256), (300, 704, 256), (64, 3392, 1280)])
def test_gemm_norm_swiglu_fp32_weight(m, f, k):
    """h = silu(rstd g + b_g) * (rstd u + b_u) with fp32 gate / up weights against fp64."""
    g = torch.Generator().manual_seed(m + f + k + 3)
    x = torch.randn(m, k, generator=g) * 1.5
    gamma = 1 + 0.1 * torch.randn(k, generator=g)
    wg = torch.randn(f, k, generator=g) * 0.05
    wu = torch.randn(f, k, generator=g) * 0.05
    bg = 0.1 * torch.randn(f, generator=g)
    bu = 0.1 * torch.randn(f, generator=g)
    hi = K().tile_matrix(K().interleave_gate_up(wg.to(torch.bfloat16), wu.to(torch.bfloat16))
                         .to(DEV))
    lo = K().tile_matrix(K().interleave_gate_up(lo_part(wg), lo_part(wu)).to(DEV))
    xd = x.double()
    rstd = 1 / torch.sqrt((xd ** 2).mean(1, keepdim=True) + 1e-5)
    a = xd * gamma.double()
    gt = rstd * (a @ wg.double().T) + bg.double()
    ut = rstd * (a @ wu.double().T) + bu.double()
    ref = gt * torch.sigmoid(gt) * ut
    # |d h| <= |d g| |dh/dg| + |d u| |dh/du|, |dh/dg| <= 1.1 |u|, |dh/du| = |silu(g)|
    sg = rstd * (a.abs() @ wg.double().abs().T)
    su = rstd * (a.abs() @ wu.double().abs().T)
    scale = 1.1 * ut.abs() * sg + (gt * torch.sigmoid(gt)).abs() * su + ref.abs()
    xt = K().tile_f32(x.to(DEV))
    for t in _tiles():
        h = torch.zeros(K().split_numel(m, f, True), device=DEV, dtype=torch.bfloat16)
        K().gemm_norm_swiglu(xt, gamma.to(DEV), 1e-5, hi, bg.to(DEV), bu.to(DEV), h, m, f, k,
                             tile=t, w_gu_lo=lo)
        torch.cuda.synchronize()
        _close(untile_split(h, m, f), ref, scale, 2 ** -15, f"tile {t}")


@pytest.mark.parametrize("m,n,k", [(37, 256, 704), (64, 1280, 3392), (500, 768, 768)])
def test_gemm_split_residual_fp32_weight(m, n, k):
    """x += (a_hi + a_lo) @ W^T + bias with W fp32, in place on the tiled residual stream."""
    g = torch.Generator().manual_seed(m + n + k + 4)
    a = torch.randn(m, k, generator=g)
    ahi = a.to(torch.bfloat16)
    alo = (a - ahi.float()).to(torch.bfloat16)
    at = K().tile_matrix(torch.cat([ahi, alo], 1).to(DEV))
    w = torch.randn(n, k, generator=g) * 0.05
    wt = K().tile_matrix(w.to(torch.bfloat16).to(DEV))
    wl = K().tile_matrix(lo_part(w).to(DEV))
    x = torch.randn(m, n, generator=g)
    bias = 0.1 * torch.randn(n, generator=g)
    ref = x.double() + a.double() @ w.double().T + bias.double()
    scale = x.double().abs() + a.double().abs() @ w.double().abs().T + bias.double().abs()
    for t in _tiles():
        xt = K().tile_f32(x.to(DEV))
        K().gemm_split_residual(at, wt, xt, bias.to(DEV), m, n, k, tile=t, w_lo=wl)
        torch.cuda.synchronize()
        _close(K().untile_f32(xt, m, n).cpu(), ref, scale, 2 ** -15, f"tile {t}")


# ------------------------------------------------------------------------------ K2, fp32 out

def _rope_setup(g, rows, H):
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    d = 64 * H
    qkv = torch.randn(rows, 3 * d, generator=g)
    rstd = 0.5 + torch.rand(rows, generator=g)
    pos = torch.randint(0, 40, (rows, 3), generator=g)
    rope = RotaryEmbedding3D(64, 30, 30, 8)
    return d, qkv, rstd, pos, rope.device_table(DEV), (30, 30, 8, rope.px, rope.py, rope.pz)


def _rope_ref(qkv, rstd, pos, H, q_scale):
    """q * q_scale, k rotated, v: [rows, H, 64] each, in fp64, from the oracle's RoPE."""
    cfg = rp.OracleConfig(d_model=64 * H, n_heads=H, n_layers=1, d_ff=64, max_x=30, max_y=30,
                          max_z=8)
    tabs = {k: v.double() for k, v in rp.rope3d_tables(cfg).items()}
    x = (qkv.double() * rstd.double()[:, None]).view(-1, 3, H, 64)
    q = rp.apply_rope3d(x[:, 0][None], pos[None], tabs, cfg)[0] * q_scale
    k = rp.apply_rope3d(x[:, 1][None], pos[None], tabs, cfg)[0]
    return q, k, x[:, 2]


@pytest.mark.parametrize("H,S,slot0,dev_slot", [(4, 33, 0, False), (12, 7, 20, True),
                                                (5, 16, 3, False)])
def test_qkv_rope_cache_fp32(H, S, slot0, dev_slot):
    g = torch.Generator().manual_seed(H * 100 + S)
    B, slots = 3, 64
    d, qkv, rstd, pos, tab, geom = _rope_setup(g, B * S, H)
    qs = 0.125 * LOG2E
    q = torch.full((B * S, d), float("nan"), device=DEV)
    kc = torch.zeros(B, H, slots, 64, device=DEV)
    vc = torch.zeros_like(kc)
    slot_dev = torch.tensor([slot0], dtype=torch.int32, device=DEV) if dev_slot else None
    K().qkv_rope_cache(qkv.to(DEV), rstd.to(DEV), pos.to(DEV), tab, geom, B, S, H, qs, q, kc, vc,
                       slot0=0 if dev_slot else slot0, slot_dev=slot_dev)
    torch.cuda.synchronize()
    rq, rk, rv = _rope_ref(qkv, rstd, pos, H, qs)
    assert torch.allclose(q.cpu().double().view(-1, H, 64), rq, rtol=1e-6, atol=1e-6)
    kk = kc.cpu().double()[:, :, slot0:slot0 + S].permute(0, 2, 1, 3).reshape(-1, H, 64)
    vv = vc.cpu().double()[:, :, slot0:slot0 + S].permute(0, 2, 1, 3).reshape(-1, H, 64)
    assert torch.allclose(kk, rk, rtol=1e-6, atol=1e-6)
    assert torch.allclose(vv, rv, rtol=1e-6, atol=1e-6)
    # nothing else of the cache is written
    other = torch.ones(slots, dtype=torch.bool)
    other[slot0:slot0 + S] = False
    assert bool((kc.cpu()[:, :, other] == 0).all()) and bool((vc.cpu()[:, :, other] == 0).all())


def test_qkv_rope_cache_packed_fp32_equals_padded():
    """The packed token list writes the same fp32 q and slots as the [batch, seq] form."""
    g = torch.Generator().manual_seed(5)
    B, S, H, slots = 3, 40, 4, 48
    d, qkv, rstd, pos, tab, geom = _rope_setup(g, B * S, H)
    kv = [0, 17, 39]
    rows = [b * S + j for b in range(B) for j in range(kv[b], S)]
    idx = torch.tensor(rows)
    qs = 0.125 * LOG2E
    q1 = torch.empty(B * S, d, device=DEV)
    kc1 = torch.zeros(B, H, slots, 64, device=DEV)
    vc1 = torch.zeros_like(kc1)
    K().qkv_rope_cache(qkv.to(DEV), rstd.to(DEV), pos.to(DEV), tab, geom, B, S, H, qs, q1, kc1,
                       vc1)
    q2 = torch.empty(len(rows), d, device=DEV)
    kc2 = torch.zeros_like(kc1)
    vc2 = torch.zeros_like(kc1)
    trow = (idx // S).to(torch.int32).to(DEV)
    tslot = (idx % S).to(torch.int32).to(DEV)
    K().qkv_rope_cache_packed(qkv[idx].to(DEV), rstd[idx].to(DEV), pos[idx].to(DEV), tab, geom,
                              trow, tslot, H, qs, q2, kc2, vc2)
    torch.cuda.synchronize()
    assert torch.equal(q2.cpu(), q1.cpu()[idx])
    for b in range(B):
        assert torch.equal(kc2[b, :, kv[b]:S], kc1[b, :, kv[b]:S])
        assert torch.equal(vc2[b, :, kv[b]:S], vc1[b, :, kv[b]:S])
        assert bool((kc2[b, :, :kv[b]] == 0).all())


# ------------------------------------------------------------------------------ K4f

def _masks(B, S, kind, g):
    m = torch.ones(B, S, dtype=torch.bool)
    if kind == "left":
        for b in range(B):
            n = [S, 0, 1, 17, S // 2][b % 5]
            m[b, :S - n] = False
    elif kind == "holes":
        m = torch.rand(B, S, generator=g) < 0.7
        m[1] = False
    return m


def _first(mask, S):
    return torch.where(mask.any(1), mask.float().argmax(1), torch.full((mask.shape[0],), S))


def _attn_close(got, ref, what=""):
    """K4f's output against fp64: the split output holds each value to 2^-17 relative, the fp32
    products and sums add ~1e-6 absolute; a bf16 rounding of q, K or V is ~2e-3 relative."""
    err = (got.double() - ref).abs()
    bound = 1e-5 + 3e-5 * ref.abs()
    ratio = (err / bound).max().item()
    assert ratio <= 1.0, f"{what} max err {err.max().item():.3e}, worst ratio {ratio:.2f}"


def _attn_ref(q_scaled, kc, vc, mask, causal, S):
    """The oracle's SDPA in fp64 on the unscaled q (the kernel's q carries 1/8 * log2(e))."""
    q = (q_scaled.double() * 8 / LOG2E).transpose(1, 2)
    return rp.attention(q, kc[:, :, :S].double(), vc[:, :, :S].double(), mask, causal)


@pytest.mark.parametrize("S", [1, 16, 37, 130, 257])
@pytest.mark.parametrize("kind", ["none", "left", "holes"])
@pytest.mark.parametrize("causal", [True, False])
def test_attn_prefill_f32(S, kind, causal):
    g = torch.Generator().manual_seed(S * 13 + len(kind) + causal)
    B, H, slots = 5, 3, S + 11
    q = torch.randn(B, S, H, 64, generator=g) * (0.125 * LOG2E) * 2.0
    kc = torch.randn(B, H, slots, 64, generator=g)
    vc = torch.randn(B, H, slots, 64, generator=g)
    mask = _masks(B, S, kind, g) if kind != "none" else None
    kv_start = None if mask is None else _first(mask, S).to(torch.int32).to(DEV)
    for tiled in (False, True):
        out = torch.full((K().tile_rows(B * S) if tiled else B * S, 2 * H * 64), float("nan"),
                         device=DEV, dtype=torch.bfloat16)
        K().attn_prefill_f32(q.to(DEV), kc.to(DEV), vc.to(DEV), B, S, H,
                             None if mask is None else mask.to(torch.uint8).to(DEV), kv_start,
                             None, B * S, causal, out, out_tiled=tiled)
        torch.cuda.synchronize()
        got = (K().untile_matrix(out, K().tile_rows(B * S), 2 * H * 64)[:B * S]
               if tiled else out)
        ref = _attn_ref(q, kc, vc, mask, causal, S)
        _attn_close(unsplit(got).view(B, S, H, 64).transpose(1, 2), ref, f"tiled={tiled}")
        # and a bf16 rounding of K would be far outside that bar
        if S >= 37 and not tiled:
            refb = _attn_ref(q, kc.to(torch.bfloat16), vc, mask, causal, S)
            assert (refb - ref).abs().max().item() > 1e-3


@pytest.mark.parametrize("causal", [True, False])
def test_attn_prefill_f32_packed_equals_padded(causal):
    """Packed query rows (queries i >= kv_start[b] at q_offset[b] + i - kv_start[b]) give the
    same bits as the [batch, seq] form for those queries; kv_start outside [0, S] clamps."""
    g = torch.Generator().manual_seed(77 + causal)
    B, H, S, slots = 4, 2, 150, 160
    q = torch.randn(B, S, H, 64, generator=g) * 0.3
    kc = torch.randn(B, H, slots, 64, generator=g)
    vc = torch.randn(B, H, slots, 64, generator=g)
    kv = torch.tensor([0, 37, 149, 5], dtype=torch.int32)
    mask = torch.ones(B, S, dtype=torch.bool)
    for b in range(B):
        mask[b, :int(kv[b])] = False
    mask[3, 60:70] = False                               # holes after kv_start
    md = mask.to(torch.uint8).to(DEV)
    ref = torch.empty(B * S, 2 * H * 64, device=DEV, dtype=torch.bfloat16)
    K().attn_prefill_f32(q.to(DEV), kc.to(DEV), vc.to(DEV), B, S, H, md, kv.to(DEV), None,
                         B * S, causal, ref)
    n = S - kv
    off = torch.cat([torch.zeros(1, dtype=torch.int32), n.cumsum(0)[:-1].to(torch.int32)])
    rows = torch.cat([torch.arange(b * S + int(kv[b]), (b + 1) * S) for b in range(B)])
    got = torch.full((int(n.sum()), 2 * H * 64), float("nan"), device=DEV, dtype=torch.bfloat16)
    K().attn_prefill_f32(q.reshape(B * S, -1)[rows].contiguous().to(DEV), kc.to(DEV), vc.to(DEV),
                         B, S, H, md, kv.to(DEV), off.to(DEV), int(n.sum()), causal, got)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), ref.cpu()[rows])
    # clamped kv_start: -1000 acts as 0, 10000 as S (no key: zeros)
    kv2 = torch.tensor([-1000, 10_000, 5, 0], dtype=torch.int32)
    out = torch.empty(B * S, 2 * H * 64, device=DEV, dtype=torch.bfloat16)
    K().attn_prefill_f32(q.to(DEV), kc.to(DEV), vc.to(DEV), B, S, H, None, kv2.to(DEV), None,
                         B * S, causal, out)
    torch.cuda.synchronize()
    m2 = torch.ones(B, S, dtype=torch.bool)
    m2[1] = False
    m2[2, :5] = False
    r2 = _attn_ref(q, kc, vc, m2, causal, S)
    _attn_close(unsplit(out).view(B, S, H, 64).transpose(1, 2), r2, "clamped kv_start")


@pytest.mark.parametrize("slots,t", [(64, 0), (300, 211), (1100, 1037)])
@pytest.mark.parametrize("with_mask", [True, False])
@pytest.mark.parametrize("split_len", [0, 128, 48])
def test_attn_decode_f32(slots, t, with_mask, split_len):
    """K4f decode against fp64, in one chunk (split_len 0: the whole cache) and in chunks of
    split_len slots merged through the workspace (chunks past t are empty)."""
    g = torch.Generator().manual_seed(slots + t + with_mask)
    split = split_len or -(-slots // 16) * 16
    nbytes = K().attn_decode_workspace_bytes(6, 4, slots, split)
    ws = torch.empty(max(nbytes // 4, 1), device=DEV) if nbytes else None
    assert (ws is None) == (split >= slots)
    B, H, S = 6, 4, min(150, t + 1)
    q = torch.randn(B, H, 64, generator=g) * 0.3
    kc = torch.randn(B, H, slots, 64, generator=g)
    vc = torch.randn(B, H, slots, 64, generator=g)
    pm = _masks(B, S, "left", g) if with_mask else None
    if with_mask and S > 20:
        pm[4, 10:20] = False                             # a hole inside the prompt
    kv_start = None if pm is None else _first(pm, S).to(torch.int32).to(DEV)
    for dev_seq, tiled in ((False, False), (True, True)):
        out = torch.empty(K().tile_rows(B) if tiled else B, 2 * H * 64, device=DEV,
                          dtype=torch.bfloat16)
        seq_dev = torch.tensor([t], dtype=torch.int32, device=DEV) if dev_seq else None
        K().attn_decode_f32(q.to(DEV), kc.to(DEV), vc.to(DEV), B, H,
                            None if pm is None else pm.to(torch.uint8).to(DEV),
                            S if pm is not None else 0, kv_start, t, seq_dev, ws, split, out,
                            tiled=tiled)
        torch.cuda.synchronize()
        got = K().untile_matrix(out, K().tile_rows(B), 2 * H * 64)[:B] if tiled else out
        keymask = torch.ones(B, t + 1, dtype=torch.bool)
        if pm is not None:
            keymask[:, :S] = pm
            if kv_start is not None:
                for b in range(B):
                    keymask[b, :int(kv_start[b])] = False
        ref = rp.attention((q.double() * 8 / LOG2E)[:, :, None], kc[:, :, :t + 1].double(),
                           vc[:, :, :t + 1].double(), keymask, causal=False)[:, :, 0]
        _attn_close(unsplit(got).view(B, H, 64), ref, f"seq_dev={dev_seq}")
