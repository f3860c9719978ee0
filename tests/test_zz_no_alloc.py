"""The no-allocation decode entry point (mdl_attn_decode_rope_noalloc, static per-GPU scratch)
against mdl_attn_decode_rope with a caller-supplied workspace: bit-identical attention output and
cache writes, on two calls in a row, the second one smaller (its splits reuse the scratch the
first call left behind)."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(seed, B, H, S, slots, t):
    from mdlarc_scale_amd.transformer import RotaryEmbedding3D

    g = torch.Generator().manual_seed(seed)
    d = 64 * H
    qkv = torch.randn(B, 3 * d, generator=g).to(DEV)
    rstd = (0.5 + torch.rand(B, generator=g)).to(DEV)
    pos = torch.randint(0, 35, (B, 3), generator=g).to(DEV)
    rope = RotaryEmbedding3D(64, 32, 32, 8)
    tab, geom = rope.device_table(DEV), (32, 32, 8, rope.px, rope.py, rope.pz)
    kc = torch.randn(B, H, slots, 64, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(B, H, slots, 64, generator=g).to(torch.bfloat16).to(DEV)
    lens = torch.randint(S // 3, S + 1, (B,), generator=g)
    pm = torch.arange(S)[None, :] >= (S - lens)[:, None]          # left padded
    pm[0, S - 20:S - 12] = False                                    # a hole inside a prompt
    kv_start = (S - lens).to(torch.int32).to(DEV)
    order = torch.argsort(kv_start).to(torch.int32)
    seq_dev = torch.tensor([t], dtype=torch.int32, device=DEV)
    return dict(qkv=qkv, rstd=rstd, pos=pos, rope_tab=tab, rope_geom=geom, q_scale=0.125,
                kc=kc, vc=vc, B=B, H=H, pm=pm.to(torch.uint8).to(DEV), S=S, kv_start=kv_start,
                order=order, seq_dev=seq_dev)


def _run(c, split_len, noalloc):
    from mdlarc_scale_amd import kernels as K

    kc, vc = c["kc"].clone(), c["vc"].clone()
    out = torch.full((c["B"], 2 * 64 * c["H"]), float("nan"), device=DEV, dtype=torch.bfloat16)
    args = (c["qkv"], c["rstd"], c["pos"], c["rope_tab"], c["rope_geom"], c["q_scale"], kc, vc,
            c["B"], c["H"], c["pm"], c["S"], c["kv_start"], 0, c["seq_dev"])
    if noalloc:
        K.attn_decode_rope_noalloc(*args, split_len, out, row_order=c["order"])
    else:
        n = K.attn_decode_workspace_bytes(c["B"], c["H"], kc.shape[2], split_len) // 4
        ws = torch.empty(n, device=DEV)
        K.attn_decode_rope(*args, ws, split_len, out, row_order=c["order"])
    torch.cuda.synchronize()
    return out, kc, vc


def test_noalloc_decode_equals_workspace_decode_twice():
    from mdlarc_scale_amd import kernels as K

    big = _case(1, B=6, H=3, S=700, slots=2600, t=2477)        # 11 splits of 256, 64-slot tiles
    small = _case(2, B=4, H=2, S=300, slots=900, t=777)        # 8 splits of 128, 32-slot tiles
    for c, split_len in ((big, 256), (small, 128)):
        need = K.attn_decode_workspace_bytes(c["B"], c["H"], c["kc"].shape[2], split_len)
        assert 0 < need <= K.DECODE_SCRATCH_BYTES
        print(f"noalloc decode: B={c['B']} H={c['H']} slots={c['kc'].shape[2]} "
              f"split_len={split_len} scratch bytes {need}", flush=True)
        ref = _run(c, split_len, noalloc=False)
        got = _run(c, split_len, noalloc=True)
        for r, x in zip(ref, got):
            assert torch.equal(r.view(torch.int16), x.view(torch.int16))
        assert not torch.isnan(got[0].float()).any()
