"""K6 (csrc/prefill_gemm.hip): the prompt projections with the RMSNorm prologue and the SwiGLU /
residual epilogues, against fp64 references of the same split-activation products, across
row / column tails, both activation layouts and every preset's shapes."""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def K():
    from mdlarc_scale_amd import kernels

    return kernels


def split(v: torch.Tensor):
    hi = v.to(torch.bfloat16)
    return hi, (v - hi.float()).to(torch.bfloat16)


def rel(a: torch.Tensor, b: torch.Tensor) -> float:
    return ((a.double() - b.double()).abs().max() / b.double().abs().max()).item()


# (m, n, k): row tails (m % 256), column tails (n % 256), every preset's K (d, d_ff)
SHAPES = [(1000, 768, 768), (333, 1408, 256), (4097, 2304, 768), (17, 768, 2048),
          (700, 1280, 3392), (256, 3072, 1024), (1, 256, 704), (1025, 4096, 2752)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_split_gemm_matches_fp64(m, n, k):
    """out = (hi + lo) . W^T to fp32 accumulation error, identical in both activation layouts."""
    g = torch.Generator().manual_seed(m + n + k)
    w = (0.05 * torch.randn(n, k, generator=g)).to(torch.bfloat16).to(DEV)
    hi, lo = split(torch.randn(m, k, generator=g).to(DEV))
    a = torch.cat([hi, lo], 1).contiguous()
    ref = (hi.double() + lo.double()) @ w.double().t()
    wt = K().tile_matrix(w)
    out = torch.full((m, n), float("nan"), device=DEV)
    K().prefill_gemm_split(a, wt, out, k)
    out_t = torch.full((m, n), float("nan"), device=DEV)
    K().prefill_gemm_split(K().tile_matrix(a), wt, out_t, k, a_tiled=True)
    torch.cuda.synchronize()
    assert rel(out, ref) < 2e-6
    assert torch.equal(out, out_t)


@pytest.mark.parametrize("m,n,k", [s for s in SHAPES if s[2] <= 2048])
def test_norm_gemm_matches_fp64(m, n, k):
    """The ln1 + qkv form: split(x * gamma) . W^T (x * gamma rounded to fp32, then split) and
    rstd = 1 / sqrt(mean(x^2) + eps)."""
    g = torch.Generator().manual_seed(7 * m + n + k)
    w = (0.05 * torch.randn(n, k, generator=g)).to(torch.bfloat16).to(DEV)
    x = torch.randn(m, k, generator=g).to(DEV)
    gam = (1 + 0.1 * torch.randn(k, generator=g)).to(DEV)
    th, tl = split(x * gam)
    ref = (th.double() + tl.double()) @ w.double().t()
    rs_ref = 1 / torch.sqrt((x.double() ** 2).mean(1) + 1e-5)
    out = torch.empty(m, n, device=DEV)
    rs = torch.empty(m, device=DEV)
    K().prefill_gemm_norm(K().tile_f32(x), gam, 1e-5, K().tile_matrix(w), out, rs, k)
    torch.cuda.synchronize()
    assert rel(out, ref) < 2e-6
    assert rel(rs, rs_ref) < 1e-6


@pytest.mark.parametrize("m,n,k", [s for s in SHAPES if s[1] % 32 == 0])
@pytest.mark.parametrize("bias", [False, True])
def test_residual_gemm_matches_fp64(m, n, k, bias):
    """x += (hi + lo) . W^T (+ bias) in place on the fp32 tile-layout residual stream; both
    activation layouts give the same x; padding rows of the tile buffer are left alone."""
    g = torch.Generator().manual_seed(3 * m + n + k + bias)
    w = (0.05 * torch.randn(n, k, generator=g)).to(torch.bfloat16).to(DEV)
    hi, lo = split(torch.randn(m, k, generator=g).to(DEV))
    a = torch.cat([hi, lo], 1).contiguous()
    x0 = torch.randn(m, n, generator=g).to(DEV)
    b = torch.randn(n, generator=g).to(DEV) if bias else None
    ref = x0.double() + (hi.double() + lo.double()) @ w.double().t()
    if bias:
        ref += b.double()
    wt = K().tile_matrix(w)
    x1 = K().tile_f32(x0)
    x1_before = x1.clone()
    K().prefill_gemm_split_residual(a, wt, x1, b, m, n, k)
    x2 = K().tile_f32(x0)
    K().prefill_gemm_split_residual(K().tile_matrix(a), wt, x2, b, m, n, k, a_tiled=True)
    torch.cuda.synchronize()
    assert rel(K().untile_f32(x1, m, n), ref) < 2e-6
    assert torch.equal(x1, x2)
    # the tile buffer's padding rows (m .. tile_rows(m) - 1) keep their values
    untiled = lambda t: K().untile_f32(t, K().tile_rows(m), n)  # noqa: E731
    assert torch.equal(untiled(x1)[m:], untiled(x1_before)[m:])


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("m,f,k", [(1000, 2048, 768), (333, 704, 256), (257, 2752, 1024),
                                   (700, 3392, 1280), (5, 2048, 768)])
def test_norm_swiglu_gemm(m, f, k, bias):
    """The ln2 + gate/up + SwiGLU form equals K3 (mdl_swiglu) applied to the same launch's gate /
    up accumulators (the E_STORE form on the interleaved weight, same main loop), bit for bit;
    and an fp64 reference to fp32 rounding.  Without biases (NULL) the epilogue adds zeros."""
    g = torch.Generator().manual_seed(m + f + k)
    wg = (0.05 * torch.randn(f, k, generator=g)).to(torch.bfloat16).to(DEV)
    wu = (0.05 * torch.randn(f, k, generator=g)).to(torch.bfloat16).to(DEV)
    wgu = K().tile_matrix(K().interleave_gate_up(wg, wu))
    x = torch.randn(m, k, generator=g).to(DEV)
    gam = (1 + 0.1 * torch.randn(k, generator=g)).to(DEV)
    bg = torch.randn(f, generator=g).to(DEV)
    bu = torch.randn(f, generator=g).to(DEV)
    if not bias:
        bg = bu = None
    xt = K().tile_f32(x)
    h = torch.empty(K().split_numel(m, f, True), dtype=torch.bfloat16, device=DEV)
    K().prefill_gemm_norm_swiglu(xt, gam, 1e-5, wgu, bg, bu, h, m, f, k)
    # unfused: gate / up accumulators (interleaved 16-column blocks) + rstd, then K3
    acc = torch.empty(m, 2 * f, device=DEV)
    rs = torch.empty(m, device=DEV)
    K().prefill_gemm_norm(xt, gam, 1e-5, wgu, acc, rs, k)
    blocks = acc.view(m, f // 16, 2, 16)
    gu = torch.cat([blocks[:, :, 0].reshape(m, f), blocks[:, :, 1].reshape(m, f)], 1).contiguous()
    h_ref = torch.empty(m, 2 * f, dtype=torch.bfloat16, device=DEV)
    K().swiglu(gu, rs, bg, bu, h_ref)
    torch.cuda.synchronize()
    assert torch.equal(K().untile_matrix(h, m, 2 * f), h_ref)
    th, tl = split(x * gam)
    t = th.double() + tl.double()
    rs64 = 1 / torch.sqrt((x.double() ** 2).mean(1) + 1e-5)
    gg = rs64[:, None] * (t @ wg.double().t())
    uu = rs64[:, None] * (t @ wu.double().t())
    if bias:
        gg, uu = gg + bg.double(), uu + bu.double()
    ref = gg / (1 + torch.exp(-gg)) * uu
    hh = K().untile_matrix(h, m, 2 * f).double()
    assert rel(hh[:, :f] + hh[:, f:], ref) < 2e-5


@pytest.mark.parametrize("m,n,k", [s for s in SHAPES if s[1] % 32 == 0])
def test_hi_only_split_forms_match_fp64(m, n, k):
    """a_parts 1: a holds hi alone ([m, k]) and the product is hi . W^T -- against fp64 to fp32
    accumulation error, in both layouts and both epilogues, and measurably apart from the split
    product (so a kernel that still added a lo term, or dropped hi, fails)."""
    g = torch.Generator().manual_seed(5 * m + n + k)
    w = (0.05 * torch.randn(n, k, generator=g)).to(torch.bfloat16).to(DEV)
    v = torch.randn(m, k, generator=g).to(DEV)
    hi, lo = split(v)
    a = hi.contiguous()
    ref = hi.double() @ w.double().t()
    assert rel(v.double() @ w.double().t(), ref) > 1e-4   # the lo term matters at this scale
    wt = K().tile_matrix(w)
    out = torch.full((m, n), float("nan"), device=DEV)
    K().prefill_gemm_split(a, wt, out, k, a_parts=1)
    out_t = torch.full((m, n), float("nan"), device=DEV)
    K().prefill_gemm_split(K().tile_matrix(a), wt, out_t, k, a_tiled=True, a_parts=1)
    x0 = torch.randn(m, n, generator=g).to(DEV)
    b = torch.randn(n, generator=g).to(DEV)
    x1 = K().tile_f32(x0)
    K().prefill_gemm_split_residual(K().tile_matrix(a), wt, x1, b, m, n, k, a_tiled=True,
                                    a_parts=1)
    x2 = K().tile_f32(x0)
    K().prefill_gemm_split_residual(a, wt, x2, b, m, n, k, a_parts=1)
    torch.cuda.synchronize()
    assert rel(out, ref) < 2e-6
    assert torch.equal(out, out_t)
    assert rel(K().untile_f32(x1, m, n), x0.double() + ref + b.double()) < 2e-6
    assert torch.equal(x1, x2)


@pytest.mark.parametrize("m,f,k", [(1000, 2048, 768), (333, 704, 256), (257, 2752, 1024),
                                   (5, 2048, 768)])
def test_norm_swiglu_parts(m, f, k):
    """a_parts 1 (gate / up of bf16(x * gamma)) against fp64 of the same hi product, h_parts 1
    (hi of h alone, [m, f]) bit-equal to the hi half of the h_parts 2 output of the same launch
    form, for both activation forms."""
    g = torch.Generator().manual_seed(3 * m + f + k)
    wg = (0.05 * torch.randn(f, k, generator=g)).to(torch.bfloat16).to(DEV)
    wu = (0.05 * torch.randn(f, k, generator=g)).to(torch.bfloat16).to(DEV)
    wgu = K().tile_matrix(K().interleave_gate_up(wg, wu))
    x = torch.randn(m, k, generator=g).to(DEV)
    gam = (1 + 0.1 * torch.randn(k, generator=g)).to(DEV)
    bg = torch.randn(f, generator=g).to(DEV)
    bu = torch.randn(f, generator=g).to(DEV)
    xt = K().tile_f32(x)
    hs = {}
    for ap in (1, 2):
        for hp in (1, 2):
            h = torch.empty(K().tile_rows(m) * hp * f, dtype=torch.bfloat16, device=DEV)
            K().prefill_gemm_norm_swiglu(xt, gam, 1e-5, wgu, bg, bu, h, m, f, k, a_parts=ap,
                                         h_parts=hp)
            hs[ap, hp] = K().untile_matrix(h, m, hp * f)
    torch.cuda.synchronize()
    for ap in (1, 2):
        assert torch.equal(hs[ap, 1], hs[ap, 2][:, :f])
    th, tl = split(x * gam)
    rs64 = 1 / torch.sqrt((x.double() ** 2).mean(1) + 1e-5)

    def swiglu64(t):
        gg = rs64[:, None] * (t @ wg.double().t()) + bg.double()
        uu = rs64[:, None] * (t @ wu.double().t()) + bu.double()
        return gg / (1 + torch.exp(-gg)) * uu

    ref_hi, ref_split = swiglu64(th.double()), swiglu64(th.double() + tl.double())
    h12 = hs[1, 2].double()
    assert rel(h12[:, :f] + h12[:, f:], ref_hi) < 2e-5
    assert rel(ref_split, ref_hi) > 1e-4   # the lo term is visible at this tolerance


def test_prefill_gemm_persistent_tiles_cover_everything():
    """More tiles than CUs (each block walks several, the load ring crossing tile boundaries):
    every output element is written once with the right value."""
    g = torch.Generator().manual_seed(11)
    m, n, k = 256 * 70 + 19, 2304, 256      # 639 tiles: each of the <= 256 blocks walks 2-3
    w = (0.05 * torch.randn(n, k, generator=g)).to(torch.bfloat16).to(DEV)
    hi, lo = split(torch.randn(m, k, generator=g).to(DEV))
    a = torch.cat([hi, lo], 1).contiguous()
    out = torch.full((m, n), float("nan"), device=DEV)
    K().prefill_gemm_split(a, K().tile_matrix(w), out, k)
    ref = (hi.double() + lo.double()) @ w.double().t()
    torch.cuda.synchronize()
    assert not bool(out.isnan().any())
    assert rel(out, ref) < 2e-6


def _rope(max_xyz=(30, 30, 8)):
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    rope = RotaryEmbedding3D(64, *max_xyz)
    return rope.device_table(DEV), (rope.max_x, rope.max_y, rope.max_z, rope.px, rope.py, rope.pz)


@pytest.mark.parametrize("packed", [True, False])
@pytest.mark.parametrize("n_heads", [4, 12])
def test_norm_qkv_equals_norm_gemm_then_k2(packed, n_heads):
    """ln1 + qkv_proj + K2 in one launch writes exactly what the E_STORE form followed by K2
    (qkv_rope_cache / _packed) writes -- q, every cache slot, rstd -- and the fp32 projection
    rows only for each row's first LEAD_QUERIES tokens from kv_start."""
    g = torch.Generator().manual_seed(n_heads * 2 + packed)
    B, S, slots = 3, 150, 170
    H, d = n_heads, 64 * n_heads
    kv = [0, 37, 149]
    if packed:   # valid tokens of each row, then one padding token (slot -1, no cache write)
        tr, ts = [], []
        for b, k0 in enumerate(kv):
            tr += [b] * (S - k0)
            ts += list(range(k0, S))
        tr.append(1)
        ts.append(-1)
        rows = len(tr)
        token_row = torch.tensor(tr, dtype=torch.int32, device=DEV)
        token_slot = torch.tensor(ts, dtype=torch.int32, device=DEV)
    else:
        rows = B * S
        token_row = token_slot = None
    x = torch.randn(rows, d, generator=g).to(DEV)
    gam = (1 + 0.1 * torch.randn(d, generator=g)).to(DEV)
    w = K().tile_matrix((0.05 * torch.randn(3 * d, d, generator=g)).to(torch.bfloat16).to(DEV))
    pos = torch.randint(0, 35, (rows, 3), generator=g).to(DEV)
    tab, geom = _rope()
    kv_dev = torch.tensor(kv, dtype=torch.int32, device=DEV)
    xt = K().tile_f32(x)
    # reference: E_STORE form, then K2
    qkv = torch.empty(rows, 3 * d, device=DEV)
    rs1 = torch.empty(rows, device=DEV)
    K().prefill_gemm_norm(xt, gam, 1e-5, w, qkv, rs1, d)
    sentinel = torch.full((B, H, slots, 64), 7.0, dtype=torch.bfloat16)
    kc1, vc1 = sentinel.clone().to(DEV), sentinel.clone().to(DEV)
    q1 = torch.empty(rows, d, dtype=torch.bfloat16, device=DEV)
    if packed:
        K().qkv_rope_cache_packed(qkv, rs1, pos, tab, geom, token_row, token_slot, H, 0.125, q1,
                                  kc1, vc1)
    else:
        K().qkv_rope_cache(qkv, rs1, pos, tab, geom, B, S, H, 0.125, q1, kc1, vc1, slot0=0)
    # fused
    kc2, vc2 = sentinel.clone().to(DEV), sentinel.clone().to(DEV)
    q2 = torch.empty(rows, d, dtype=torch.bfloat16, device=DEV)
    rs2 = torch.empty(rows, device=DEV)
    lead = torch.full((rows, 3 * d), float("nan"), device=DEV)
    K().prefill_gemm_norm_qkv(xt, gam, 1e-5, w, rows, H, rs2, lead, K().LEAD_QUERIES, kv_dev, pos,
                              tab, geom, 0.125, q2, kc2, vc2, token_row=token_row,
                              token_slot=token_slot, seq=0 if packed else S)
    torch.cuda.synchronize()
    assert torch.equal(rs1, rs2)
    assert torch.equal(q1, q2)
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    # lead rows: slot in [kv_start[b], kv_start[b] + 64)
    if packed:
        rb, sl = token_row.long().cpu(), token_slot.long().cpu()
    else:
        rb = torch.arange(rows) // S
        sl = torch.arange(rows) % S
    ks = torch.tensor(kv)[rb]
    is_lead = (sl >= ks) & (sl - ks < K().LEAD_QUERIES)
    assert int(is_lead.sum()) > 0
    li = is_lead.to(DEV)
    assert torch.equal(lead[li], qkv[li])
    assert bool(lead[~li].isnan().all())


def test_split_gemm_at_config2_size_against_hipblaslt():
    """At config 2's packed prefill size (268,148 rows, the qkv projection's N = 2304, K = 768)
    K6 agrees with hipBLASLt on the [W | W] operand (an independent GEMM, fp32 accumulation in
    another order) to fp32 rounding over every element, and with fp64 on sampled rows."""
    from mdlarc_scale_amd.engine import gemm_f32, pack_split_weight

    g = torch.Generator(device=DEV).manual_seed(3)
    m, n, k = 268_148, 2304, 768
    w = (0.05 * torch.randn(n, k, generator=g, device=DEV)).to(torch.bfloat16)
    v = torch.randn(m, k, generator=g, device=DEV)
    hi, lo = split(v)
    a = torch.cat([hi, lo], 1).contiguous()
    del v, lo
    out = torch.empty(m, n, device=DEV)
    K().prefill_gemm_split(K().tile_matrix(a), K().tile_matrix(w), out, k, a_tiled=True)
    ref = torch.empty(m, n, device=DEV)
    gemm_f32(a, pack_split_weight(w, DEV), ref)
    torch.cuda.synchronize()
    scale = ref.abs().max()
    assert float((out - ref).abs().max() / scale) < 2e-6
    rows = torch.randint(0, m, (512,), generator=g, device=DEV)
    aa = a[rows].double()
    sub = (aa[:, :k] + aa[:, k:]) @ w.double().t()
    assert float((out[rows].double() - sub).abs().max() / sub.abs().max()) < 2e-6
