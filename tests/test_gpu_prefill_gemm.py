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


@pytest.mark.parametrize("m,f,k", [(1000, 2048, 768), (333, 704, 256), (257, 2752, 1024),
                                   (700, 3392, 1280), (5, 2048, 768)])
def test_norm_swiglu_gemm(m, f, k):
    """The ln2 + gate/up + SwiGLU form equals K3 (mdl_swiglu) applied to the same launch's gate /
    up accumulators (the E_STORE form on the interleaved weight, same main loop), bit for bit;
    and an fp64 reference to fp32 rounding."""
    g = torch.Generator().manual_seed(m + f + k)
    wg = (0.05 * torch.randn(f, k, generator=g)).to(torch.bfloat16).to(DEV)
    wu = (0.05 * torch.randn(f, k, generator=g)).to(torch.bfloat16).to(DEV)
    wgu = K().tile_matrix(K().interleave_gate_up(wg, wu))
    x = torch.randn(m, k, generator=g).to(DEV)
    gam = (1 + 0.1 * torch.randn(k, generator=g)).to(DEV)
    bg = torch.randn(f, generator=g).to(DEV)
    bu = torch.randn(f, generator=g).to(DEV)
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
    gg = rs64[:, None] * (t @ wg.double().t()) + bg.double()
    uu = rs64[:, None] * (t @ wu.double().t()) + bu.double()
    ref = gg / (1 + torch.exp(-gg)) * uu
    hh = K().untile_matrix(h, m, 2 * f).double()
    assert rel(hh[:, :f] + hh[:, f:], ref) < 2e-5


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
