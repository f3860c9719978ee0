"""HIP execution engine of the TinyTransformer inference path.

Dataflow per layer (M token rows, d channels, F ffn width; fp32 residual stream x), written in
its unfused form:

    xs = split(x * g1), rstd                                                    [M, 2d] bf16
    qkv = xs @ [W_qkv|W_qkv]^T       (bf16 x bf16 -> fp32)                       [M, 3d] fp32
    K2: q = rope(rstd*q)/8 -> [M, d] bf16; k, v = rope(rstd*k), rstd*v -> bf16 cache slots
    attn = K4(q, cache)              (prefill: MFMA flash; decode: split-K)      [M, 2d] bf16
           (prefill: the first 64 queries of each row recomputed exactly in fp32, K4c)
    x += attn @ [W_out|W_out]^T
    gu = split(x * g2) @ [W_gu|W_gu]^T  (gate and up concatenated)               [M, 2F] fp32
    h = split(silu(rstd*g + b_g) * (rstd*u + b_u))                               [M, 2F] bf16
    x += h @ [W_down|W_down]^T + b_down
  final: logits = lm_head(ln_f(x)) and greedy argmax                <- lm_head kernel

Every projection runs on a hand-written MFMA GEMM that reads the tiled copy of W (read once,
not as [W | W], in the MFMA tile layout) and takes the small kernels into its prologue and
epilogue; x (fp32) lives in the fp32 tile layout.  Per layer:

    q, K, V = K2(split(x * g1) @ Wqkv^T)           <- norm_qkv (ln1 in the prologue, K2 in the
                                                      epilogue)
    attn = K4(...)                                 (tiled output)
    x += attn @ Wo^T                                <- split_residual
    h = split(silu(rstd*g + b_g) * (rstd*u + b_u)), g / u = split(x * g2) @ Wg^T / Wu^T
                                                    <- norm_swiglu (ln2 in the prologue)
    x += h @ Wd^T + b_down                          <- split_residual

At decode (M = batch rows) these are K5 launches (tall thin GEMMs: the weights are the traffic);
for a prompt (M = batch * prompt length) they are K6 launches (persistent 256 x 256 tiles).
The head kernel takes ln_f itself.  Shapes outside K6's limits (d_model > 2048, or a width that
is not a multiple of 32) run the prompt's projections on hipBLASLt against [W | W] with K1,
add_rmsnorm, K2 and K3 as separate passes.

"split" stores a GEMM input as a hi|lo pair of bf16 (hi = bf16(v), lo = bf16(v - hi)); against a
weight packed as [W | W] the bf16 MFMA GEMM then sees the activation to ~2^-17 instead of 2^-9.
Rounding every GEMM operand and output to a single bf16 puts the final logits 3e-2 away from the
fp32 reference on the reference-initialised presets; with split inputs and fp32 outputs the only
bf16 roundings left are the weights (shared with the reference's bf16 configurations) and the
q/K/V operands of attention, and the logits land within about 1e-2.

Weights are packed once per model version (bf16 [W | W] GEMM operands, fp32 gains / biases /
head); the embedding tables are read live from the module parameters, because test-time
adaptation edits ``example_embed.weight.data`` between calls.

Two forms, chosen by the model's parameter dtype as the reference chooses its cache dtype
(``next(model.parameters()).dtype``, src/inference.py:522):

* bf16 form (a bf16 model: the reference's configurations 2-4): everything above.
* fp32 form (a model with fp32 parameters: configuration 0).  The reference then keeps fp32
  weights, an fp32 cache and fp32 attention, so this form does too: each weight W goes to the
  K5 GEMMs as w = bf16(W) plus w_lo = bf16(W - w) (a third product a_hi . w_lo per k-step, W to
  ~2^-17), q / K / V and the cache are fp32 (K2 with fp32 outputs) and the attention is K4f
  (fp32 MFMA).  Per layer of a prompt or a decode step:

    qkv, rstd = split(x * g1) @ (w + w_lo)^T                     <- K5 norm (E_STORE), fp32 out
    q, K, V = K2(qkv) in fp32, K / V into the fp32 cache        <- qkv_rope_cache (fp32)
    attn = K4f(q, cache)                                         <- attn_prefill_f32 / decode_f32
    then the three K5 launches of the bf16 decode form, each with its w_lo.

  The prompt's projections run on K5 too (K6 has no room in LDS for a second weight stage).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import kernels as K
from .transformer import TinyTransformer, attention_q_scale, softmax_scale

START, NEWLINE, IO_SEP, END = 10, 11, 12, 13
GRID_MAX_X, GRID_MAX_Y = 30, 29     # GridStateUpdater defaults (src/inference.py:107)


def gemm_f32(a: torch.Tensor, w2: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[M, N] (fp32) = a[M, 2K] (split bf16) @ w2[N, 2K]^T (bf16 [W | W]) on hipBLASLt with
    fp32 accumulation and an unrounded fp32 result."""
    return torch.ops.aten.mm.dtype_out(a, w2.t(), torch.float32, out=out)


def tiles_supported(d_model: int, d_ff: int) -> bool:
    """K5 with tiled operands needs every projection's K (d_model, d_ff) to be a multiple of 32;
    all reference presets are."""
    return d_model % 32 == 0 and d_ff % 32 == 0


def zero_tiled_rows(buf: torch.Tensor, r0: int, r1: int, cols: int) -> None:
    """Zero rows [r0, r1) of a bf16 [rows, cols] matrix in the MFMA tile layout: each row is
    cols / 8 chunks of 8 contiguous elements (tile_off of include/mdlarc_hip.h)."""
    m = torch.arange(r0, r1, device=buf.device)[:, None]
    q = torch.arange(cols // 8, device=buf.device)[None, :]
    chunk = 64 * ((m >> 4) * (cols >> 5) + (q >> 2)) + 16 * (q & 3) + (m & 15)
    buf.view(-1, 8)[chunk.reshape(-1)] = 0


# Activation parts of the bf16 form's prompt MLP on K6 (2: split hi | lo, as every other
# projection; 1: the lo term dropped, as the reference's bf16 model rounds a projection's input
# to bf16).  PROMPT_GATE_UP_PARTS is the gate / up input's (bf16(ln2(x)) at 1),
# PROMPT_DOWN_PARTS the down input's (h stored as hi alone at 1).  Measured at config 2 (one
# layer's launches): 1 for both takes gate/up 3.21 -> 2.35 ms and down 1.52 -> 1.01 ms, but the
# config-2 decode logits move from 4.8e-3 to 2.9e-2 of the fp32 oracle (over the 2e-2 bar);
# down alone gives 1.2e-2.  Both stay at 2 -- the parity margin is worth more than the 2-5 ms.
PROMPT_GATE_UP_PARTS = 2
PROMPT_DOWN_PARTS = 2


def prompt_gemms_fused(d_model: int, d_ff: int) -> bool:
    """K6 runs a prompt's projections (RMSNorms and residual adds fused in) when the tiled
    weights exist and the normed inputs fit its LDS copy of gamma; every reference preset does.
    Otherwise the prompt path runs hipBLASLt on [W | W] with separate norm / SwiGLU passes."""
    return tiles_supported(d_model, d_ff) and d_model <= K.PREFILL_NORM_MAX_K


def model_form(model: TinyTransformer) -> str:
    """"fp32" for a model whose parameters are fp32, "bf16" for a bf16 model: the dtype the
    reference keeps its cache and attention in (``next(model.parameters()).dtype``,
    src/inference.py:522, :544)."""
    dt = next(model.parameters()).dtype
    if dt == torch.float32:
        return "fp32"
    if dt == torch.bfloat16:
        return "bf16"
    raise TypeError(f"mdlarc_scale_amd runs float32 and bfloat16 models (got {dt})")


def split_weight_lo(w: torch.Tensor) -> torch.Tensor:
    """bf16(W - bf16(W)): the low part of an fp32 weight (exact in fp32; W = hi + lo to
    ~2^-17 relative)."""
    w = w.detach().float()
    return (w - w.to(torch.bfloat16).float()).to(torch.bfloat16)


def pack_split_weight(w: torch.Tensor, device: torch.device) -> torch.Tensor:
    """bf16 [W | W] ([N, 2K]) for a split-activation GEMM input (see gemm_f32)."""
    wb = w.detach().to(device=device, dtype=torch.bfloat16)
    return torch.cat([wb, wb], dim=1).contiguous()


class PackedWeights:
    """Device copies of the weights in the layout the kernels and GEMMs consume.  ``f32`` marks
    the fp32 form: the tiled weights then come with their low parts (``*_lo``) and no [W | W]
    copies are kept (the fp32 form runs every projection on K5)."""

    def __init__(self, model: TinyTransformer, device: torch.device):
        cfg = model.config
        self.f32 = model_form(model) == "fp32"
        f32 = lambda t: t.detach().to(device=device, dtype=torch.float32).contiguous()  # noqa: E731
        pk = lambda t: pack_split_weight(t, device)  # noqa: E731
        self.tiles_ok = tiles_supported(cfg.d_model, cfg.d_ff)
        if self.f32 and not self.tiles_ok:
            raise ValueError("the fp32 form runs its projections on K5, which needs d_model and "
                             f"d_ff multiples of 32 (got {cfg.d_model}, {cfg.d_ff}); run the "
                             "model in bfloat16 instead")
        self.qkv, self.out, self.gu, self.down = [], [], [], []
        self.ln1, self.ln2, self.b_gate, self.b_up, self.b_down = [], [], [], [], []
        w_qkv, w_out, w_gu, w_down = [], [], [], []
        for blk in model.blocks:
            w_qkv.append(blk.attn.qkv_proj.weight)
            w_out.append(blk.attn.out_proj.weight)
            w_gu.append((blk.ffn.fc_gate.weight, blk.ffn.fc_up.weight))
            w_down.append(blk.ffn.fc_down.weight)
            if not self.f32:
                self.qkv.append(pk(blk.attn.qkv_proj.weight))
                self.out.append(pk(blk.attn.out_proj.weight))
                self.gu.append(pk(torch.cat([blk.ffn.fc_gate.weight, blk.ffn.fc_up.weight], 0)))
                self.down.append(pk(blk.ffn.fc_down.weight))
            self.ln1.append(f32(blk.ln1.weight))
            self.ln2.append(f32(blk.ln2.weight))
            self.b_gate.append(f32(blk.ffn.fc_gate.bias))
            self.b_up.append(f32(blk.ffn.fc_up.bias))
            self.b_down.append(f32(blk.ffn.fc_down.bias))
        # K5 / K6: each weight once, in the MFMA tile layout; gate / up with their 16-row blocks
        # interleaved (the SwiGLU runs in that GEMM's epilogue).  The fp32 form adds the tiled
        # low parts.
        n_l = len(model.blocks)
        self.qkv_lo = self.out_lo = self.gu_lo = self.down_lo = [None] * n_l
        self.qkv_t = self.out_t = self.gu_t = self.down_t = None
        if self.tiles_ok:
            hi = lambda w: w.detach().to(device=device, dtype=torch.bfloat16)  # noqa: E731
            lo = lambda w: split_weight_lo(w.to(device))  # noqa: E731
            tile = lambda w: K.tile_matrix(w.contiguous())  # noqa: E731
            gu = lambda f, pair: K.interleave_gate_up(f(pair[0]), f(pair[1]))  # noqa: E731
            self.qkv_t = [tile(hi(w)) for w in w_qkv]
            self.out_t = [tile(hi(w)) for w in w_out]
            self.gu_t = [K.tile_matrix(gu(hi, p)) for p in w_gu]
            self.down_t = [tile(hi(w)) for w in w_down]
            if self.f32:
                self.qkv_lo = [tile(lo(w)) for w in w_qkv]
                self.out_lo = [tile(lo(w)) for w in w_out]
                self.gu_lo = [K.tile_matrix(gu(lo, p)) for p in w_gu]
                self.down_lo = [tile(lo(w)) for w in w_down]
        self.ln_f = f32(model.ln_f.weight)
        self.head = f32(model.lm_head.weight)
        rope = model.blocks[0].attn.rope
        self.rope_tab = rope.device_table(device)
        self.rope_geom = (rope.max_x, rope.max_y, rope.max_z, rope.px, rope.py, rope.pz)
        self.eps = cfg.norm_eps


@dataclass
class Scratch:
    """Activation buffers for M rows (reused across layers).  xs / attn / h are split bf16 GEMM
    inputs (2x the channel count; in the MFMA tile layout, whole 16-row blocks, when ``tiled``);
    qkv / delta / gu are fp32 GEMM outputs.  The fused forms (``tiled`` decode on K5, ``fused``
    prompts on K6) form xs inside the GEMMs and keep no delta / gu: those are empty there.  On
    K6, h holds PROMPT_DOWN_PARTS parts."""

    x: torch.Tensor
    xs: torch.Tensor
    rstd: torch.Tensor
    qkv: torch.Tensor
    q: torch.Tensor
    attn: torch.Tensor
    delta: torch.Tensor
    gu: torch.Tensor
    h: torch.Tensor
    rows: int = 0
    tiled: bool = False
    fused: bool = False
    f32: bool = False

    @staticmethod
    def alloc(rows: int, d: int, d_ff: int, device: torch.device,
              tiled: bool = False, fused: bool = False, f32: bool = False) -> "Scratch":
        """``tiled``: the decode form -- x in the fp32 tile layout and attn / h in the bf16 one
        (whole 16-row blocks); the RMSNorms run inside the K5 launches (``HipEngine._mlp``).
        ``fused``: the prompt form on K6 -- the same layouts; the RMSNorms run inside the K6
        launches.  ``f32``: the fp32 form (prompt or decode) -- the ``tiled`` layouts on K5,
        q in fp32, qkv the fp32 projection output of every row."""
        e = lambda *s, dt=torch.bfloat16: torch.empty(*s, dtype=dt, device=device)  # noqa: E731
        f = torch.float32
        tiled = tiled or f32
        split_gemm = not (tiled or fused)               # hipBLASLt path: xs, delta, gu
        sr = rows if split_gemm else K.tile_rows(rows)  # rows of the tiled activations
        fused = fused and not f32
        h_parts = PROMPT_DOWN_PARTS if fused else 2
        return Scratch(x=e(sr, d, dt=f), xs=e(sr if split_gemm else 0, 2 * d),
                       rstd=e(rows, dt=f), qkv=e(rows, 3 * d, dt=f),
                       q=e(rows, d, dt=f if f32 else torch.bfloat16),
                       attn=e(sr, 2 * d), delta=e(rows if split_gemm else 0, d, dt=f),
                       gu=e(rows if split_gemm else 0, 2 * d_ff, dt=f), h=e(sr, h_parts * d_ff),
                       rows=rows, tiled=tiled, fused=fused, f32=f32)

    @staticmethod
    def for_prompt(rows: int, cfg, device: torch.device, f32: bool) -> "Scratch":
        """Scratch of a prompt pass: the fp32 form, or the bf16 form on K6 when the model's
        shapes fit it (hipBLASLt otherwise)."""
        if f32:
            return Scratch.alloc(rows, cfg.d_model, cfg.d_ff, device, f32=True)
        return Scratch.alloc(rows, cfg.d_model, cfg.d_ff, device,
                             fused=prompt_gemms_fused(cfg.d_model, cfg.d_ff))


@dataclass
class PackedPrompt:
    """The tokens of a left-padded [B, S] prompt batch with the padding left out.

    Row b contributes its tokens j in [kv_start[b], S) (slots j of its cache row), in order, at
    packed rows q_offset[b] .. q_offset[b] + S - kv_start[b] - 1; ``n_valid`` rows in all.  The
    reference reads its logits at index lengths-1 of each left-padded row, which is a padding
    token when a row is shorter than its padding: such a token is appended after the valid ones
    (cache slot -1, never written).  A padding query sees no key, so its attention output is 0
    and its hidden state depends on its own embedding only; the extra rows reproduce exactly
    that.  ``head_row[b]`` is the packed row whose logits row b reports."""

    gather: torch.Tensor       # int32 [T]: flat index b*S + j into the [B, S] inputs
    token_row: torch.Tensor    # int32 [T]
    token_slot: torch.Tensor   # int32 [T] (-1 on the extra rows)
    q_offset: torch.Tensor     # int32 [B]
    head_row: torch.Tensor     # int32 [B]
    n_valid: int
    n_tokens: int


def pack_prompt(kv_start: np.ndarray, last_row: np.ndarray, batch: int, seq: int,
                device: torch.device) -> PackedPrompt:
    """PackedPrompt of a batch whose rows start at ``kv_start`` (first valid index) and report
    logits at flat row ``last_row`` (b*S + index), both host int arrays of length ``batch``.
    The per-row quantities are computed on the host; the per-token lists are built on
    ``device`` from them (no host copy of the token lists)."""
    if batch * seq >= 2 ** 31:
        raise ValueError("packed prompts index [B, S] with int32; B*S must stay below 2^31")
    kv = np.clip(np.asarray(kv_start, dtype=np.int64), 0, seq)
    last = np.asarray(last_row, dtype=np.int64) - np.arange(batch, dtype=np.int64) * seq
    if last.size and (last.min() < 0 or last.max() >= seq):
        raise ValueError("last_row must lie inside its own row")
    n = seq - kv
    off = np.concatenate([[0], np.cumsum(n)[:-1]]).astype(np.int64)
    n_valid = int(n.sum())
    inside = last >= kv
    extra = np.nonzero(~inside)[0]
    head = np.where(inside, off + last - kv, 0)
    head[extra] = n_valid + np.arange(extra.size)
    total = n_valid + extra.size
    e = extra.size
    small = torch.from_numpy(np.concatenate(
        [kv, n, off, head, extra * seq + last[extra], extra]).astype(np.int64)).to(device)
    kv_d, n_d, off_d = small[:batch], small[batch:2 * batch], small[2 * batch:3 * batch]
    head_d = small[3 * batch:4 * batch]
    ex_gather, ex_row = small[4 * batch:4 * batch + e], small[4 * batch + e:4 * batch + 2 * e]
    rows = torch.repeat_interleave(torch.arange(batch, device=device), n_d,
                                   output_size=n_valid)
    slot = torch.arange(n_valid, device=device) - off_d[rows] + kv_d[rows]
    i32 = torch.int32
    return PackedPrompt(
        gather=torch.cat([rows * seq + slot, ex_gather]).to(i32),
        token_row=torch.cat([rows, ex_row]).to(i32),
        token_slot=torch.cat([slot, torch.full((e,), -1, dtype=torch.int64,
                                               device=device)]).to(i32),
        q_offset=off_d.to(i32), head_row=head_d.to(i32), n_valid=n_valid, n_tokens=total)


DECODE_MIN_BLOCKS = 2048   # 8 four-wave blocks per CU on 256 CUs


def choose_split_len(n_bh: int, slots: int) -> int:
    """Slots per decode-attention work item (a multiple of 128).  One chunk per (row, head) once
    B*H alone gives DECODE_MIN_BLOCKS blocks -- splitting further only adds the partial-merge
    pass (measured at config 2: 3,072 (b, h) pairs, one chunk each, is the fastest) -- and just
    enough chunks to reach that count for small batches."""
    n_split = max(1, -(-DECODE_MIN_BLOCKS // max(n_bh, 1)))
    per = -(-slots // n_split)
    return max(128, -(-per // 128) * 128)


class HipEngine:
    def __init__(self, model: TinyTransformer):
        self.model = model
        self._packed: PackedWeights | None = None
        self._sig: tuple | None = None

    def invalidate(self) -> None:
        self._packed, self._sig = None, None

    def _signature(self) -> tuple:
        return tuple((p.data_ptr(), p._version, p.dtype, p.device)
                     for n, p in self.model.named_parameters()
                     if not n.startswith(("token_embed", "example_embed")))

    def packed(self, device: torch.device) -> PackedWeights:
        sig = self._signature()
        if self._packed is None or sig != self._sig:
            with torch.no_grad():
                self._packed = PackedWeights(self.model, device)
            self._sig = sig
        return self._packed

    # -- helpers -------------------------------------------------------------------------------
    @property
    def cfg(self):
        return self.model.config

    def _tables(self):
        m = self.model
        return m.token_embed.weight.detach(), m.example_embed.weight.detach()

    @staticmethod
    def _check_device(t: torch.Tensor) -> torch.device:
        if not t.is_cuda:
            raise RuntimeError("mdlarc_scale_amd runs the inference path on a ROCm GPU; move the "
                               f"model and inputs to a GPU device (got {t.device})")
        return t.device

    def _validate_ids(self, ids: torch.Tensor, ex: torch.Tensor | None) -> None:
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= self.cfg.vocab_size):
            raise IndexError("input_ids out of range of the token embedding")
        if ex is not None and ex.numel() and (int(ex.min()) < 0 or
                                              int(ex.max()) >= self.cfg.num_examples):
            raise IndexError("example_ids out of range of the example embedding")

    # -- full-sequence layers (prefill / forward) ------------------------------------------------
    def run_prompt(self, W: PackedWeights, ids: torch.Tensor, pos: torch.Tensor,
                   ex_ids: torch.Tensor | None, key_mask: torch.Tensor | None,
                   kv_start: torch.Tensor | None, causal: bool, kv_layers,
                   sc: Scratch, row_holes: torch.Tensor | None = None) -> None:
        """Run every layer over [B, S] tokens; leaves the final residual in ``sc.x``.
        ``kv_layers(li)`` returns the (k, v) [B, H, slots, 64] views to write slots [0, S).
        ``row_holes`` (uint8 [B], from grid_init) lets the attention skip reading the key mask of
        the rows where it is the run [kv_start, S)."""
        cfg = self.cfg
        B, S = ids.shape
        H, d = cfg.n_heads, cfg.d_model
        tok, ex = self._tables()
        use_ex = ex_ids if (ex_ids is not None and cfg.use_example_embedding) else None
        fused = sc.fused   # K6: ln1 runs in the qkv launch, so the embedding writes x only
        nx = fused or sc.f32   # ln1 inside the projection: the embedding writes x only
        K.embed_rmsnorm(ids.reshape(-1), use_ex, tok, ex if use_ex is not None else None, S,
                        W.ln1[0], W.eps, sc.x, None if nx else sc.xs,
                        None if nx else sc.rstd, tiled=nx)
        qs = softmax_scale(d // H)          # the exact lead pass (K4c)
        qa = attention_q_scale(d // H)      # q for the attention kernels (log2-domain softmax)
        for li in range(cfg.n_layers):
            kc, vc = kv_layers(li)
            if sc.f32:
                # fp32 form: projection on K5 with the low weight part, K2 into the fp32 cache,
                # K4f (the attention is exact, so no lead pass)
                K.gemm_norm(sc.x, W.ln1[li], W.eps, W.qkv_t[li], sc.qkv, sc.rstd, d,
                            w_lo=W.qkv_lo[li])
                K.qkv_rope_cache(sc.qkv, sc.rstd, pos, W.rope_tab, W.rope_geom, B, S, H, qa,
                                 sc.q, kc, vc, slot0=0)
                K.attn_prefill_f32(sc.q, kc, vc, B, S, H, key_mask, kv_start, None, B * S,
                                   causal, sc.attn, out_tiled=True)
                self._mlp(W, li, sc)
                continue
            if fused:   # ln1 + qkv_proj + K2 in one launch (fp32 qkv only for the lead rows)
                K.prefill_gemm_norm_qkv(sc.x, W.ln1[li], W.eps, W.qkv_t[li], B * S, H, sc.rstd,
                                        sc.qkv, K.LEAD_QUERIES if causal else 0, kv_start, pos,
                                        W.rope_tab, W.rope_geom, qa, sc.q, kc, vc, seq=S)
            else:
                gemm_f32(sc.xs, W.qkv[li], sc.qkv)
                K.qkv_rope_cache(sc.qkv, sc.rstd, pos, W.rope_tab, W.rope_geom, B, S, H, qa,
                                 sc.q, kc, vc, slot0=0)
            K.attn_prefill(sc.q, kc, vc, B, S, H, key_mask, kv_start, causal, sc.attn,
                           out_tiled=fused, row_holes=row_holes)
            if causal:
                K.attn_prefill_lead(sc.qkv, sc.rstd, pos, W.rope_tab, W.rope_geom, qs, B, S, H,
                                    key_mask, kv_start, None, B * S, sc.attn, out_tiled=fused)
            self._mlp(W, li, sc)

    def run_packed(self, W: PackedWeights, ids: torch.Tensor, pos: torch.Tensor,
                   ex_ids: torch.Tensor | None, key_mask: torch.Tensor | None,
                   kv_start: torch.Tensor, pk: PackedPrompt, kv_layers, sc: Scratch,
                   row_holes: torch.Tensor | None = None) -> None:
        """``run_prompt`` (causal) over the packed tokens ``pk`` of the [B, S] batch ``ids`` /
        ``pos``: every GEMM and elementwise kernel sees pk.n_tokens rows instead of B*S.  K/V of
        the valid tokens go to their slots; leaves the final residual in ``sc.x`` (packed rows).
        ``sc`` must hold pk.n_tokens rows; ``row_holes`` as in ``run_prompt``."""
        cfg = self.cfg
        B, S = ids.shape
        H, d = cfg.n_heads, cfg.d_model
        tok, ex = self._tables()
        use_ex = ex_ids is not None and cfg.use_example_embedding
        ids_p = ids.reshape(-1).index_select(0, pk.gather)
        pos_p = pos.reshape(-1, 3).index_select(0, pk.gather)
        ex_p = ex_ids.reshape(-1).index_select(0, pk.token_row) if use_ex else None
        fused = sc.fused
        nx = fused or sc.f32   # ln1 inside the projection: the embedding writes x only
        K.embed_rmsnorm(ids_p, ex_p, tok, ex if use_ex else None, 1, W.ln1[0], W.eps, sc.x,
                        None if nx else sc.xs, None if nx else sc.rstd, tiled=nx)
        if pk.n_tokens > pk.n_valid:   # padding queries: no visible key, attention output 0
            if nx:
                zero_tiled_rows(sc.attn, pk.n_valid, pk.n_tokens, 2 * d)
            else:
                sc.attn[pk.n_valid:pk.n_tokens].zero_()
        qs = softmax_scale(d // H)          # the exact lead pass (K4c)
        qa = attention_q_scale(d // H)      # q for the attention kernels (log2-domain softmax)
        for li in range(cfg.n_layers):
            kc, vc = kv_layers(li)
            if sc.f32:   # fp32 form (see run_prompt)
                K.gemm_norm(sc.x, W.ln1[li], W.eps, W.qkv_t[li], sc.qkv, sc.rstd, d,
                            w_lo=W.qkv_lo[li])
                K.qkv_rope_cache_packed(sc.qkv, sc.rstd, pos_p, W.rope_tab, W.rope_geom,
                                        pk.token_row, pk.token_slot, H, qa, sc.q, kc, vc)
                K.attn_prefill_f32(sc.q, kc, vc, B, S, H, key_mask, kv_start, pk.q_offset,
                                   pk.n_tokens, True, sc.attn, out_tiled=True)
                self._mlp(W, li, sc)
                continue
            if fused:
                K.prefill_gemm_norm_qkv(sc.x, W.ln1[li], W.eps, W.qkv_t[li], pk.n_tokens, H,
                                        sc.rstd, sc.qkv, K.LEAD_QUERIES, kv_start, pos_p,
                                        W.rope_tab, W.rope_geom, qa, sc.q, kc, vc,
                                        token_row=pk.token_row, token_slot=pk.token_slot)
            else:
                gemm_f32(sc.xs, W.qkv[li], sc.qkv)
                K.qkv_rope_cache_packed(sc.qkv, sc.rstd, pos_p, W.rope_tab, W.rope_geom,
                                    pk.token_row, pk.token_slot, H, qa, sc.q, kc, vc)
            K.attn_prefill_packed(sc.q, kc, vc, B, S, H, key_mask, kv_start, pk.q_offset,
                                  pk.n_valid, True, sc.attn, out_tiled=fused,
                                  row_holes=row_holes)
            K.attn_prefill_lead(sc.qkv, sc.rstd, pos_p, W.rope_tab, W.rope_geom, qs, B, S, H,
                                key_mask, kv_start, pk.q_offset, pk.n_tokens, sc.attn,
                                out_tiled=fused)
            self._mlp(W, li, sc)

    def _mlp(self, W: PackedWeights, li: int, sc: Scratch) -> None:
        """out_proj + residual, ln2, SwiGLU MLP + residual, next norm (shared by both phases)."""
        cfg = self.cfg
        d, F = cfg.d_model, cfg.d_ff
        if sc.fused:
            # prompt on K6: residual adds in the out / down epilogues, ln2 in the gate / up
            # prologue with the SwiGLU in its epilogue; the next layer's ln1 runs in its qkv
            # launch (_qkv) and ln_f in the head kernel.  The MLP's inputs carry
            # PROMPT_GATE_UP_PARTS / PROMPT_DOWN_PARTS parts.
            m, parts = sc.rows, PROMPT_DOWN_PARTS
            K.prefill_gemm_split_residual(sc.attn, W.out_t[li], sc.x, None, m, d, d, a_tiled=True)
            K.prefill_gemm_norm_swiglu(sc.x, W.ln2[li], W.eps, W.gu_t[li], W.b_gate[li],
                                       W.b_up[li], sc.h, m, F, d, a_parts=PROMPT_GATE_UP_PARTS,
                                       h_parts=parts)
            K.prefill_gemm_split_residual(sc.h, W.down_t[li], sc.x, W.b_down[li], m, d, F,
                                          a_tiled=True, a_parts=parts)
            return
        if sc.tiled:
            # decode: three K5 launches, the residual adds in the epilogues and ln2 in the
            # gate / up prologue; the next layer's ln1 runs in its qkv launch (gemm_norm) and
            # ln_f in the head kernel
            # (the fp32 form adds each weight's low part)
            K.gemm_split_residual(sc.attn, W.out_t[li], sc.x, None, sc.rows, d, d,
                                  w_lo=W.out_lo[li])
            K.gemm_norm_swiglu(sc.x, W.ln2[li], W.eps, W.gu_t[li], W.b_gate[li], W.b_up[li],
                               sc.h, sc.rows, F, d, w_gu_lo=W.gu_lo[li])
            K.gemm_split_residual(sc.h, W.down_t[li], sc.x, W.b_down[li], sc.rows, d, F,
                                  w_lo=W.down_lo[li])
            return
        gemm_f32(sc.attn, W.out[li], sc.delta)
        K.add_rmsnorm(sc.x, sc.delta, None, W.ln2[li], W.eps, sc.xs, sc.rstd)
        gemm_f32(sc.xs, W.gu[li], sc.gu)
        K.swiglu(sc.gu, sc.rstd, W.b_gate[li], W.b_up[li], sc.h)
        gemm_f32(sc.h, W.down[li], sc.delta)
        last = li + 1 == cfg.n_layers
        K.add_rmsnorm(sc.x, sc.delta, W.b_down[li], W.ln_f if last else W.ln1[li + 1], W.eps,
                      None if last else sc.xs, sc.rstd)

    @staticmethod
    def key_mask_and_start(attention_mask: torch.Tensor | None, dev: torch.device, S: int):
        """The [B, S] key mask as uint8 and each row's first valid position (S when it has
        none): the attention skips the keys before it and the lead-query pass starts there.
        (None, None) without a mask."""
        if attention_mask is None:
            return None, None
        mask = attention_mask.to(device=dev, dtype=torch.bool).to(torch.uint8).contiguous()
        first = mask.to(torch.int32).argmax(1)
        kv_start = torch.where(mask.bool().any(1), first, torch.full_like(first, S)).to(
            torch.int32).contiguous()
        return mask, kv_start

    @torch.no_grad()
    def forward(self, ids: torch.Tensor, pos: torch.Tensor, ex_ids: torch.Tensor | None,
                attention_mask: torch.Tensor | None, is_causal: bool) -> torch.Tensor:
        """``TinyTransformer.forward`` on the HIP path: logits [B, S, V] in the model dtype."""
        return self.forward_f32(ids, pos, ex_ids, attention_mask, is_causal).to(
            self.model.lm_head.weight.dtype)

    @torch.no_grad()
    def forward_f32(self, ids, pos, ex_ids=None, attention_mask=None, is_causal=True):
        dev = self._check_device(ids)
        cfg = self.cfg
        B, S = ids.shape
        ids = ids.to(torch.int64).contiguous()
        pos = pos.to(device=dev, dtype=torch.int64).contiguous()
        if ex_ids is not None:
            ex_ids = ex_ids.to(device=dev, dtype=torch.int64).contiguous()
        self._validate_ids(ids, ex_ids)
        W = self.packed(dev)
        mask, kv_start = self.key_mask_and_start(attention_mask, dev, S)
        H = cfg.n_heads
        kbuf = torch.empty(B, H, S, 64, dtype=torch.float32 if W.f32 else torch.bfloat16,
                           device=dev)
        vbuf = torch.empty_like(kbuf)
        sc = Scratch.for_prompt(B * S, cfg, dev, W.f32)
        self.run_prompt(W, ids, pos, ex_ids, mask, kv_start, is_causal, lambda li: (kbuf, vbuf),
                        sc)
        logits = torch.empty(B * S, cfg.vocab_size, dtype=torch.float32, device=dev)
        K.lm_head(sc.x, None, B * S, W.ln_f, W.eps, W.head, logits, None, x_tiled=sc.tiled or
                  sc.fused)
        return logits.view(B, S, cfg.vocab_size)


def engine_for(model: TinyTransformer) -> HipEngine:
    eng = getattr(model, "_hip_engine", None)
    if eng is None or eng.model is not model:
        eng = HipEngine(model)
        object.__setattr__(model, "_hip_engine", eng)
    return eng
