"""Batched static-KV-cache generation -- drop-in for src/inference.py of
shyampathak22/mdlARC_scale.

``generate_output`` keeps the reference's signature and token-for-token semantics
(src/inference.py:487-628), including its quirks:
  * the first token and the initial grid state come from index ``lengths-1`` of each row even
    when the batch is left-padded (src/inference.py:185-191, :420-424);
  * rows that emitted END keep generating; the loop stops before a step once every row has
    emitted END (:589-595, :622-623);
  * the total length is capped at ``max_seq_len`` and an over-long prompt comes back unchanged.

The greedy loop keeps all state on the GPU: each decode step is a fixed launch sequence (grid
step -> embedding -> layers -> head/argmax -> commit) with the cache slot and output column in a
device counter, and the host reads the per-row END step only every ``SYNC_EVERY`` steps, then
trims the output to where the reference would have stopped.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import kernels as K
from .data import (
    DIHEDRAL_TRANSFORMS,
    END_TOKEN_ID,
    IO_SEP_TOKEN_ID,
    NEWLINE_TOKEN_ID,
    START_TOKEN_ID,
    apply_color_perm_grid,
    compute_positions_3d,
    decode_output_grid,
    encode_example,
    generate_color_permutations,
)
from .engine import GRID_MAX_X, GRID_MAX_Y, HipEngine, PackedWeights, Scratch, choose_split_len
from .engine import pack_prompt
from .engine import engine_for, gemm_f32, model_form, tiles_supported
from .transformer import TinyTransformer, attention_q_scale

SYNC_EVERY = 8
# Greedy constrained decoding applies the constraints inside the head kernel (and replays the
# captured step); False routes it through the host torch restatement between launches instead.
FUSED_CONSTRAINTS = True
# The fused augmentation caller builds its prompts on the device (mdl_build_prompts); False
# tokenises them on the host.
DEVICE_PROMPTS = True
# Replay greedy decode steps from one captured HIP graph (False: launch every kernel from the host
# each step; same kernels, same results).
USE_GRAPHS = True
# Prefill runs over the prompt tokens without their left padding (packed rows); False runs every
# layer over the whole padded [B, S] batch.  Logits and cache contents agree to fp32 rounding (the
# GEMMs see a different row count).
PACKED_PREFILL = True
# Decode steps run their projections on K5 over activations and weights in the MFMA tile
# layouts, with the RMSNorms, residual adds and SwiGLU inside those launches (five per layer);
# False runs hipBLASLt and the separate norm / SwiGLU kernels on row-major activations.  Logits
# agree to fp32 rounding.
DECODE_TILED = True


# =============================================================================================
# decoding constraints (src/inference.py:36-43, :285-364)
# =============================================================================================

@dataclass(frozen=True)
class DecodingConstraints:
    palette_mask: torch.Tensor | None = None
    target_shape: torch.Tensor | None = None
    palette_penalty: float = 2.0
    shape_penalty: float = 2.0
    disallow_tokens: tuple[int, ...] = (START_TOKEN_ID, IO_SEP_TOKEN_ID)


def _per_row(t: torch.Tensor | None, batch: int, width: int, device) -> torch.Tensor | None:
    """[batch, width] view of a constraint tensor, broadcasting a single row; None if the
    batch sizes are incompatible (the reference then ignores the constraint)."""
    if t is None:
        return None
    t = t.to(device).reshape(-1, width)
    if t.shape[0] == batch:
        return t
    return t.expand(batch, width) if t.shape[0] == 1 else None


def apply_logit_constraints(logits: torch.Tensor, gx: torch.Tensor, gy: torch.Tensor,
                            constraints: DecodingConstraints | None) -> torch.Tensor:
    """Soft palette / shape penalties on logits [B, V] (src/inference.py:285-364), in place.
    ``gx``/``gy`` are the grid state after consuming the current input token."""
    if constraints is None:
        return logits
    B = logits.shape[0]
    for tok in constraints.disallow_tokens:
        logits[:, tok] = float("-inf")
    pal = _per_row(constraints.palette_mask, B, 10, logits.device)
    if pal is not None:
        logits[:, :10] -= (~pal.bool()).to(logits.dtype) * constraints.palette_penalty
    shape = _per_row(constraints.target_shape, B, 2, logits.device)
    if shape is not None:
        th, tw = shape[:, 0], shape[:, 1]
        has = (th >= 0) & (tw >= 0)
        x, y = gx.long(), gy.long()
        pen = constraints.shape_penalty
        row_full = (has & (x >= tw)).to(logits.dtype) * pen
        row_open = (has & (x < tw)).to(logits.dtype) * pen
        past_end = (has & (y >= th)).to(logits.dtype) * pen
        # one subtraction per penalty, in the reference's order (it rounds each separately)
        logits[:, :10] -= row_full[:, None]
        logits[:, NEWLINE_TOKEN_ID] -= row_open
        logits[:, :10] -= past_end[:, None]
        logits[:, NEWLINE_TOKEN_ID] -= past_end
    return logits


def _head_constraints(c: DecodingConstraints, st) -> K.HeadConstraints:
    """The constraints of one generation in the head kernels' device form, bound to the decode
    state's grid position (the state after the current token, as at src/inference.py:586-611).
    Shapes normalise as in the host path: a single row broadcasts, other mismatches drop that
    constraint."""
    dev = st.gx.device
    return K.HeadConstraints(c.disallow_tokens, _per_row(c.palette_mask, st.B, 10, dev),
                             c.palette_penalty, _per_row(c.target_shape, st.B, 2, dev),
                             st.gx, st.gy, c.shape_penalty)


def _pick(logits: torch.Tensor, temperature: float, top_k: int | None) -> torch.Tensor:
    """Greedy argmax or (top-k) multinomial sampling (src/inference.py:573-583)."""
    if temperature <= 0:
        return logits.argmax(-1)
    lt = logits / max(temperature, 1e-6)
    if top_k is not None and top_k > 0:
        vals, idx = torch.topk(lt, min(top_k, lt.shape[-1]), dim=-1)
        probs = torch.zeros_like(lt).scatter_(1, idx, F.softmax(vals, dim=-1))
    else:
        probs = F.softmax(lt, dim=-1)
    return torch.multinomial(probs, 1).squeeze(-1)


# =============================================================================================
# cache and grid state (API of src/inference.py:51-221)
# =============================================================================================

class StaticKVCache:
    """Preallocated [n_layers, 2, B, H, max_seq_len, head_dim] cache (src/inference.py:51-96) in
    the model's parameter dtype, as the reference allocates it (src/inference.py:522, :544):
    bf16 for a bf16 model, fp32 for an fp32 model (the fp32 form's attention reads it in fp32)."""

    def __init__(self, batch_size: int, max_seq_len: int, n_layers: int, n_heads: int,
                 head_dim: int, device: torch.device, dtype: torch.dtype = torch.bfloat16, *,
                 zero: bool = True):
        """``zero=False`` skips the initial fill: the generation path writes every slot before
        any kernel reads it (prefill writes [kv_start, S) of each row, each decode step writes
        its slot first, and no kernel reads a row's slots before its kv_start)."""
        self.batch_size, self.max_seq_len, self.n_layers = batch_size, max_seq_len, n_layers
        self.seq_len = 0
        alloc = torch.zeros if zero else torch.empty
        self.cache = alloc(n_layers, 2, batch_size, n_heads, max_seq_len, head_dim,
                           device=device, dtype=dtype)

    def reset(self) -> None:
        self.cache.zero_()
        self.seq_len = 0

    def layer(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.cache[layer_idx, 0], self.cache[layer_idx, 1]

    def update(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor):
        n = k.size(2)
        end = self.seq_len + n
        self.cache[layer_idx, 0, :, :, self.seq_len:end] = k
        self.cache[layer_idx, 1, :, :, self.seq_len:end] = v
        return self.cache[layer_idx, 0, :, :, :end], self.cache[layer_idx, 1, :, :, :end]

    def advance(self, n: int = 1) -> None:
        self.seq_len += n


class GridStateUpdater:
    """Per-row (x, y, in_output) decode-position tracker (src/inference.py:104-168), stepped by
    the ``mdl_grid_step`` kernel on the GPU."""

    def __init__(self, batch_size: int, device: torch.device, max_x: int = GRID_MAX_X,
                 max_y: int = GRID_MAX_Y):
        self.device, self.max_x, self.max_y = torch.device(device), max_x, max_y
        HipEngine._check_device(torch.empty(0, device=self.device))
        self.gx = torch.zeros(batch_size, dtype=torch.int32, device=self.device)
        self.gy = torch.zeros(batch_size, dtype=torch.int32, device=self.device)
        self.gio = torch.ones(batch_size, dtype=torch.uint8, device=self.device)
        self._pos = torch.empty(batch_size, 3, dtype=torch.int64, device=self.device)

    @property
    def x(self) -> torch.Tensor:
        return self.gx.long()

    @property
    def y(self) -> torch.Tensor:
        return self.gy.long()

    @property
    def in_output(self) -> torch.Tensor:
        return self.gio.bool()

    def reset(self) -> None:
        self.gx.zero_()
        self.gy.zero_()
        self.gio.fill_(1)

    def set_state(self, x: torch.Tensor, y: torch.Tensor, in_output: torch.Tensor) -> None:
        self.gx.copy_(x.to(self.device).clamp(-2**31, 2**31 - 1).to(torch.int32))
        self.gy.copy_(y.to(self.device).clamp(-2**31, 2**31 - 1).to(torch.int32))
        self.gio.copy_(in_output.to(self.device).to(torch.uint8))

    def update(self, tokens: torch.Tensor) -> torch.Tensor:
        tok = tokens.to(self.device, torch.int64).reshape(-1).contiguous()
        K.grid_step(tok, self.gx, self.gy, self.gio, self._pos, None, self.max_x, self.max_y)
        return self._pos.clone()


def _derive_initial_state_from_prompt(input_ids: torch.Tensor, positions_3d: torch.Tensor,
                                      attention_mask: torch.Tensor | None, max_x: int,
                                      max_y: int):
    """Grid state after the prompt, read at index lengths-1 (src/inference.py:171-221)."""
    B, S = input_ids.shape
    dev = input_ids.device
    mask = None if attention_mask is None else attention_mask.to(dev).bool().to(
        torch.uint8).contiguous()
    gx = torch.empty(B, dtype=torch.int32, device=dev)
    gy = torch.empty_like(gx)
    io = torch.empty(B, dtype=torch.uint8, device=dev)
    K.grid_init(input_ids.to(torch.int64).contiguous(),
                positions_3d.to(dev, torch.int64).contiguous(), mask, gx, gy, io, None, None,
                max_x, max_y)
    return gx.long(), gy.long(), io.bool()


# =============================================================================================
# generation
# =============================================================================================

@dataclass
class DecodeState:
    """Device-resident state of one batched generation."""

    B: int
    S: int
    total: int
    ex: torch.Tensor            # [B] int64 example ids
    pmask: torch.Tensor         # [B, S] uint8 prompt mask
    kv_start: torch.Tensor      # [B] int32 first valid prompt slot
    last_row: torch.Tensor      # [B] int32 prefill row the first token is read from
    holes: torch.Tensor         # [B] uint8 1 if the prompt mask has holes after kv_start
    order: torch.Tensor         # [B] int32 rows by descending prompt length (attention dispatch)
    gx: torch.Tensor
    gy: torch.Tensor
    gio: torch.Tensor
    pos: torch.Tensor           # [B, 3] int64 position of the current input token
    tok: torch.Tensor           # [B] int64 current token
    counters: torch.Tensor      # int32 [2]: cache slot of the current token, output column
    out_ids: torch.Tensor       # [B, total] int64
    finish: torch.Tensor        # [B] int32 first generated index of END, -1 if none
    logits: torch.Tensor        # [B, V] fp32
    cache: StaticKVCache
    sc: Scratch
    ws: torch.Tensor | None
    split_len: int


class Generator:
    """Prefill + decode loop of ``generate_output`` on the HIP kernels."""

    def __init__(self, model: TinyTransformer):
        self.model = model
        self.eng = engine_for(model)

    def prepare(self, input_ids, positions_3d, example_ids, prompt_mask, total,
                row_shift: torch.Tensor | None = None) -> DecodeState:
        """Device state for generating up to ``total`` columns.  ``row_shift`` (int32 [B]) maps
        each row's lengths-1 index from the narrower batch the reference padded it in (see
        ``mdl_grid_init``)."""
        cfg = self.model.config
        dev = input_ids.device
        B, S = input_ids.shape
        H, hd = cfg.n_heads, cfg.d_model // cfg.n_heads
        f32 = model_form(self.model) == "fp32"
        cache = StaticKVCache(B, total, cfg.n_layers, H, hd, dev,
                              dtype=torch.float32 if f32 else torch.bfloat16, zero=False)
        pmask = prompt_mask.to(torch.uint8).contiguous()
        i32 = lambda: torch.empty(B, dtype=torch.int32, device=dev)  # noqa: E731
        gx, gy, kv_start, last_row = i32(), i32(), i32(), i32()
        gio = torch.empty(B, dtype=torch.uint8, device=dev)
        holes = torch.empty(B, dtype=torch.uint8, device=dev)
        K.grid_init(input_ids, positions_3d, pmask, gx, gy, gio, kv_start, last_row,
                    row_holes=holes, row_shift=row_shift)
        # longest rows first: the decode-attention launch dispatches them before the short ones
        order = torch.argsort(kv_start, stable=True).to(torch.int32)
        split = choose_split_len(B * H, total)
        nbytes = K.attn_decode_workspace_bytes(B, H, total, split)
        ws = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=dev) if nbytes else None
        out_ids = torch.empty(B, total, dtype=torch.int64, device=dev)
        out_ids[:, :S] = input_ids
        return DecodeState(
            B=B, S=S, total=total, ex=example_ids, pmask=pmask, kv_start=kv_start,
            last_row=last_row, holes=holes, order=order, gx=gx, gy=gy, gio=gio,
            pos=torch.empty(B, 3, dtype=torch.int64, device=dev),
            tok=torch.empty(B, dtype=torch.int64, device=dev),
            counters=torch.tensor([S - 1, S], dtype=torch.int32, device=dev),
            out_ids=out_ids, finish=torch.full((B,), -1, dtype=torch.int32, device=dev),
            logits=torch.empty(B, cfg.vocab_size, dtype=torch.float32, device=dev),
            cache=cache, ws=ws,
            sc=Scratch.alloc(B, cfg.d_model, cfg.d_ff, dev, f32=f32,
                             tiled=DECODE_TILED and tiles_supported(cfg.d_model, cfg.d_ff)),
            split_len=split)

    def prefill(self, st: DecodeState, W: PackedWeights, input_ids, positions_3d,
                cons: K.HeadConstraints | None = None) -> None:
        """``_prefill`` (src/inference.py:383-424): all layers over the prompt, K/V into slots
        [0, S), logits of row lengths-1 into ``st.logits`` and its argmax into ``st.tok``
        (after ``cons``, the fused logit constraints, when given)."""
        cfg = self.model.config
        dev = input_ids.device
        if PACKED_PREFILL:
            # one small device->host read of the row starts; the padding then costs nothing
            starts = torch.stack([st.kv_start, st.last_row]).cpu().numpy()
            pk = pack_prompt(starts[0], starts[1], st.B, st.S, dev)
            sc = Scratch.for_prompt(pk.n_tokens, cfg, dev, W.f32)
            self.eng.run_packed(W, input_ids, positions_3d, st.ex, st.pmask, st.kv_start, pk,
                                st.cache.layer, sc, row_holes=st.holes)
            head_row = pk.head_row
        else:
            sc = Scratch.for_prompt(st.B * st.S, cfg, dev, W.f32)
            self.eng.run_prompt(W, input_ids, positions_3d, st.ex, st.pmask, st.kv_start, True,
                                st.cache.layer, sc, row_holes=st.holes)
            head_row = st.last_row
        K.lm_head(sc.x, head_row, st.B, W.ln_f, W.eps, W.head, st.logits, st.tok, cons,
                  x_tiled=sc.fused or sc.tiled)
        st.cache.seq_len = st.S

    def _embed_inputs(self, st: DecodeState):
        cfg = self.model.config
        tok_tab, ex_tab = self.eng._tables()
        use_ex = st.ex if cfg.use_example_embedding else None
        return tok_tab, (ex_tab if use_ex is not None else None), use_ex

    def _layers(self, st: DecodeState, W: PackedWeights) -> None:
        """Every layer of ``_decode_step`` (src/inference.py:437-456) for the embedded token in
        ``st.sc``: K/V of the new token go to slot counters[0]; leaves the residual in sc.x."""
        cfg = self.model.config
        sc, B = st.sc, st.B
        H = cfg.n_heads
        qs = attention_q_scale(cfg.d_model // H)   # q for the attention kernels
        slot = st.counters[0:1]
        for li in range(cfg.n_layers):
            kc, vc = st.cache.layer(li)
            if sc.f32:
                # fp32 form: projection with the low weight part, K2 of the token into slot t
                # of the fp32 cache, K4f over slots [kv_start, t]
                K.gemm_norm(sc.x, W.ln1[li], W.eps, W.qkv_t[li], sc.qkv, sc.rstd, cfg.d_model,
                            w_lo=W.qkv_lo[li])
                K.qkv_rope_cache(sc.qkv, sc.rstd, st.pos, W.rope_tab, W.rope_geom, B, 1, H, qs,
                                 sc.q, kc, vc, slot_dev=slot)
                K.attn_decode_f32(sc.q, kc, vc, B, H, st.pmask, st.S, st.kv_start, 0, slot,
                                  st.ws, st.split_len, sc.attn, tiled=True)
            elif sc.tiled:
                # ln1 in the projection's prologue, K2 (RoPE, q scale, K/V into slot t) in its
                # epilogue; the attention reads q and the cache
                K.gemm_norm_qkv(sc.x, W.ln1[li], W.eps, W.qkv_t[li], B, H, None, st.pos,
                                W.rope_tab, W.rope_geom, qs, sc.q, kc, vc, slot_dev=slot)
                K.attn_decode(sc.q, kc, vc, B, H, st.pmask, st.S, st.kv_start, 0, slot, st.ws,
                              st.split_len, sc.attn, row_holes=st.holes, row_order=st.order,
                              tiled=True)
            else:
                gemm_f32(sc.xs, W.qkv[li], sc.qkv)
                # RMSNorm scale + split + 3D RoPE + cache write fused into the attention launch
                K.attn_decode_rope(sc.qkv, sc.rstd, st.pos, W.rope_tab, W.rope_geom, qs, kc, vc,
                                   B, H, st.pmask, st.S, st.kv_start, 0, slot, st.ws,
                                   st.split_len, sc.attn, row_holes=st.holes, row_order=st.order,
                                   tiled=False)
            self.eng._mlp(W, li, sc)

    def decode_layers(self, st: DecodeState, W: PackedWeights, want_logits: bool) -> None:
        """``_decode_step`` (src/inference.py:427-459) for the token in ``st.tok`` at the
        position in ``st.pos``; K/V go to slot counters[0]; greedy token back into ``st.tok``
        (the host-launched path of sampling / constrained decoding)."""
        sc = st.sc
        tok_tab, ex_tab, use_ex = self._embed_inputs(st)
        t = sc.tiled
        K.embed_rmsnorm(st.tok, use_ex, tok_tab, ex_tab, 1, W.ln1[0], W.eps, sc.x,
                        None if t else sc.xs, None if t else sc.rstd, tiled=t)
        self._layers(st, W)
        K.lm_head(sc.x, None, st.B, W.ln_f, W.eps, W.head, st.logits if want_logits else None,
                  st.tok, x_tiled=t)

    def greedy_step(self, st: DecodeState, W: PackedWeights, stop_on_end: bool,
                    cons: K.HeadConstraints | None = None) -> None:
        """One full device-side decode step of greedy generation: grid position + embedding,
        the layers, then LM head (+ logit constraints) + argmax + commit."""
        sc = st.sc
        tok_tab, ex_tab, use_ex = self._embed_inputs(st)
        t = sc.tiled
        K.decode_embed(st.tok, use_ex, tok_tab, ex_tab, W.ln1[0], W.eps, st.gx, st.gy, st.gio,
                       st.pos, st.counters, sc.x, None if t else sc.xs, None if t else sc.rstd,
                       tiled=t)
        self._layers(st, W)
        K.decode_head(sc.x, W.ln_f, W.eps, W.head, None, st.tok, st.out_ids, 0, st.counters,
                      st.finish if stop_on_end else None, st.S, END_TOKEN_ID, cons, x_tiled=t)

    def capture_greedy(self, st: DecodeState, W: PackedWeights, stop_on_end: bool,
                       cons: K.HeadConstraints | None = None) -> torch.cuda.CUDAGraph:
        """Record ``greedy_step`` into a HIP graph.  Every buffer it touches is preallocated in
        ``st`` and the cache slot / output column advance through ``st.counters`` on the device,
        so one recording replays as every later step.  Capturing launches nothing; the caller
        must have run the step eagerly once (library handles and GEMM workspaces initialised).
        The step records no memset nodes.

        The capture runs on a side stream through ``capture_begin`` / ``capture_end`` rather than
        the ``torch.cuda.graph`` context, which first empties torch's allocator cache: returning
        that memory (the prefill's scratch) to the driver leaves every later HBM-bound kernel of
        the process about 4% slower on this platform (measured on the decode attention's read
        pattern; compute-bound kernels are unaffected)."""
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            g.capture_begin()
            try:
                self.greedy_step(st, W, stop_on_end, cons)
            finally:
                g.capture_end()
        torch.cuda.current_stream().wait_stream(side)
        return g


def generate_output(model: TinyTransformer, input_ids: torch.Tensor, positions_3d: torch.Tensor,
                    example_ids: torch.Tensor | None = None,
                    attention_mask: torch.Tensor | None = None, max_new_tokens: int = 900,
                    temperature: float = 0.0, top_k: int | None = None, stop_on_end: bool = True,
                    use_compile: bool = False,
                    constraints: DecodingConstraints | None = None) -> torch.Tensor:
    """Autoregressive generation with a static KV cache; returns [B, S + generated] int64
    (src/inference.py:487-628).  ``use_compile`` is accepted for API compatibility; the HIP
    path needs no compiler."""
    del use_compile
    model.eval()
    cfg = model.config
    B, S = input_ids.shape
    # argument checks and the early return in the reference's order (src/inference.py:527-537)
    if attention_mask is not None and tuple(attention_mask.shape) != (B, S):
        raise ValueError("attention_mask must have shape [batch, seq_len]")
    total = min(S + max_new_tokens, cfg.max_seq_len)
    if total - S <= 0:
        return input_ids
    out_ids, finish, produced = _generate(model, input_ids, positions_3d, example_ids,
                                          attention_mask, total, temperature, top_k, stop_on_end,
                                          constraints)
    g = produced
    if stop_on_end:
        fin = finish.cpu()
        if bool((fin >= 0).all()):
            g = min(g, int(fin.max()) + 1)
    return out_ids[:, :S + g]


def _generate(model: TinyTransformer, input_ids, positions_3d, example_ids, attention_mask,
              total: int, temperature: float, top_k: int | None, stop_on_end: bool,
              constraints: DecodingConstraints | None, row_shift: torch.Tensor | None = None):
    """Prefill + decode of up to ``total - S`` tokens.  Returns (out_ids [B, S + produced],
    finish [B] int32 = generated index of each row's first END or -1, produced).  The loop stops
    early once every row has emitted END (checked every SYNC_EVERY greedy steps), so
    ``produced`` may exceed the reference's count; callers trim."""
    B, S = input_ids.shape
    max_new = total - S
    eng = engine_for(model)
    dev = eng._check_device(input_ids)
    ids = input_ids.to(torch.int64).contiguous()
    pos = positions_3d.to(device=dev, dtype=torch.int64).contiguous()
    ex = (torch.zeros(B, dtype=torch.int64, device=dev) if example_ids is None
          else example_ids.to(device=dev, dtype=torch.int64).contiguous())
    if attention_mask is None:
        prompt_mask = torch.ones(B, S, dtype=torch.bool, device=dev)
    else:
        prompt_mask = attention_mask.to(device=dev, dtype=torch.bool)
    eng._validate_ids(ids, ex)
    if row_shift is not None:
        row_shift = row_shift.to(device=dev, dtype=torch.int32).contiguous()
    gen = Generator(model)
    with torch.no_grad():
        W = eng.packed(dev)
        st = gen.prepare(ids, pos, ex, prompt_mask, total, row_shift)
        # sampling runs on the host between launches; greedy decoding (constrained or not) is
        # one device-side step replayed from a captured graph, constraints fused into the head
        eager = temperature > 0 or (constraints is not None and not FUSED_CONSTRAINTS)
        cons = None if (eager or constraints is None) else _head_constraints(constraints, st)
        gen.prefill(st, W, ids, pos, cons)
        if eager:
            apply_logit_constraints(st.logits, st.gx, st.gy, constraints)
            st.tok.copy_(_pick(st.logits, temperature, top_k))
        K.decode_commit(st.tok, st.out_ids, S, None, st.finish if stop_on_end else None, S,
                        END_TOKEN_ID)
        produced = 1
        graph = None
        for step in range(1, max_new):
            if stop_on_end and (eager or step % SYNC_EVERY == 0) and bool((st.finish >= 0).all()):
                break
            if eager:
                K.grid_step(st.tok, st.gx, st.gy, st.gio, st.pos, st.counters)
                gen.decode_layers(st, W, want_logits=True)
                apply_logit_constraints(st.logits, st.gx, st.gy, constraints)
                st.tok.copy_(_pick(st.logits, temperature, top_k))
                K.decode_commit(st.tok, st.out_ids, 0, st.counters,
                                st.finish if stop_on_end else None, S, END_TOKEN_ID)
            elif graph is not None:
                graph.replay()
            else:
                gen.greedy_step(st, W, stop_on_end, cons)
                if USE_GRAPHS and step + 1 < max_new:
                    graph = gen.capture_greedy(st, W, stop_on_end, cons)
            produced += 1
    return st.out_ids[:, :S + produced], st.finish, produced


# =============================================================================================
# task-level helpers (src/inference.py:631-1008)
# =============================================================================================

def predict_grid(model: TinyTransformer, input_grids, output_grids, test_input, device,
                 example_id: int = 0, max_output_tokens: int = 900, temperature: float = 0.0,
                 top_k: int | None = None, use_compile: bool = False,
                 constraints: DecodingConstraints | None = None):
    """One prompt -> predicted output grid or None (src/inference.py:631-694)."""
    model.eval()
    toks: list[int] = []
    for inp, out in zip(input_grids, output_grids, strict=True):
        toks += encode_example(inp, out)
    toks += encode_example(test_input, None)
    ids = torch.tensor([toks], dtype=torch.long, device=device)
    pos = torch.from_numpy(compute_positions_3d(toks))[None].to(device)
    ex = torch.tensor([example_id], dtype=torch.long, device=device)
    with torch.no_grad():
        out_ids = generate_output(model, ids, pos, ex, max_new_tokens=max_output_tokens,
                                  temperature=temperature, top_k=top_k, stop_on_end=True,
                                  constraints=constraints)
    seq = out_ids[0].cpu().tolist()
    seps = [i for i, t in enumerate(seq) if t == IO_SEP_TOKEN_ID]
    return decode_output_grid(seq[seps[-1]:]) if seps else None


def _grid_shape(grid) -> tuple[int, int] | None:
    if not grid or not grid[0]:
        return None
    w = len(grid[0])
    return (len(grid), w) if all(len(r) == w for r in grid) else None


def _infer_output_shape(task: dict) -> tuple[int, int] | None:
    shapes = [_grid_shape(p.get("output")) for p in task.get("train", [])]
    if not shapes or any(s is None for s in shapes) or len(set(shapes)) != 1:
        return None
    return shapes[0]


def _collect_palette(task: dict, test_idx: int, include_test_input: bool = False) -> set[int]:
    cols: set[int] = set()
    grids = [p.get(k) for p in task.get("train", []) for k in ("input", "output")]
    if include_test_input and task.get("test"):
        grids.append(task["test"][test_idx]["input"])
    for g in grids:
        for row in g or []:
            cols.update(int(v) for v in row)
    return cols


def _transform_shape(shape, dihedral_idx: int):
    if shape is None:
        return None
    return (shape[1], shape[0]) if dihedral_idx in (1, 3, 6, 7) else shape


@dataclass
class _Variant:
    tokens: list[int] | None     # None when the prompt is built on the device
    dihedral: int
    perm: tuple[int, ...] | None
    palette: set[int] | None
    shape: tuple[int, int] | None
    perm_row: int = 0            # row of generate_color_permutations(num_color_perms, 42)


def _build_variants(task, test_idx, use_train_examples, num_color_perms, num_samples,
                    constrain, base_palette, base_shape, tokenize: bool = True) -> list[_Variant]:
    """Every dihedral x colour-permutation prompt, in the reference's order
    (src/inference.py:794-827); ``tokenize=False`` keeps only the variant's description (the
    device builds the prompts, ``_device_prompts``)."""
    pairs = task["train"] if use_train_examples else []
    test_in = task["test"][test_idx]["input"]
    perms = generate_color_permutations(num_color_perms, seed=42)
    out: list[_Variant] = []
    for di, fn in enumerate(DIHEDRAL_TRANSFORMS):
        ins = [fn(p["input"]) for p in pairs]
        outs = [fn(p["output"]) for p in pairs]
        tin = fn(test_in)
        shape = _transform_shape(base_shape, di) if constrain else None
        for pi in range(num_color_perms):
            perm = perms[pi]
            palette = None
            if base_palette is not None:
                palette = {int(perm[c]) for c in base_palette} if pi > 0 else base_palette
            ptuple = tuple(int(v) for v in perm) if pi > 0 else None
            if not tokenize:
                out += [_Variant(None, di, ptuple, palette, shape, pi) for _ in range(num_samples)]
                continue
            if pi > 0:
                ins_p = [apply_color_perm_grid(g, perm) for g in ins]
                outs_p = [apply_color_perm_grid(g, perm) for g in outs]
                tin_p = apply_color_perm_grid(tin, perm)
            else:
                ins_p, outs_p, tin_p = ins, outs, tin
            toks: list[int] = []
            for a, b in zip(ins_p, outs_p, strict=True):
                toks += encode_example(a, b)
            toks += encode_example(tin_p, None)
            out += [_Variant(toks, di, ptuple, palette, shape, pi) for _ in range(num_samples)]
    return out


def _task_grids(task, test_idx, use_train_examples) -> list | None:
    """[in0, out0, ..., test_in] as int arrays, or None when a grid is not rectangular (only the
    host tokeniser handles those)."""
    pairs = task["train"] if use_train_examples else []
    grids = [g for p in pairs for g in (p["input"], p["output"])] + [task["test"][test_idx]["input"]]
    out = []
    for g in grids:
        if g and any(len(r) != len(g[0]) for r in g):
            return None
        out.append(np.asarray(g, dtype=np.int64).reshape(len(g), len(g[0]) if g else 0))
    return out


def _device_prompts(grids: list, variants: list[_Variant], num_color_perms: int, device):
    """The variants' prompts built on the device (mdl_build_prompts), left-padded: ids, pos,
    mask and the per-row prompt lengths.  A transposing dihedral swaps a grid's h and w; a grid
    of h x w is h*(w+1) tokens; each pair adds START / IO_SEP / END, the test START / IO_SEP."""
    swaps = (1, 3, 6, 7)
    n_pairs = (len(grids) - 1) // 2
    seg = lambda g, d: (g.shape[1] * (g.shape[0] + 1) if d in swaps       # noqa: E731
                        else g.shape[0] * (g.shape[1] + 1))
    lengths = [3 * n_pairs + 2 + sum(seg(g, v.dihedral) for g in grids) for v in variants]
    S = max(lengths)
    offs = np.cumsum([0] + [g.size for g in grids])
    cells = np.concatenate([g.reshape(-1) for g in grids] + [np.zeros(1, np.int64)]) % 10
    meta = np.array([[offs[i], g.shape[0], g.shape[1]] for i, g in enumerate(grids)], np.int32)
    perms = generate_color_permutations(num_color_perms, seed=42).astype(np.int32)
    var = np.array([[v.dihedral, v.perm_row] for v in variants], dtype=np.int32)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)   # noqa: E731
    B = len(variants)
    ids = torch.empty(B, S, dtype=torch.int64, device=device)
    pos = torch.empty(B, S, 3, dtype=torch.int64, device=device)
    mask = torch.empty(B, S, dtype=torch.uint8, device=device)
    K.build_prompts(to(cells.astype(np.uint8)), to(meta), to(var), to(perms),
                    to(np.array(lengths, dtype=np.int32)), ids, pos, mask)
    return ids, pos, mask.bool(), lengths


def left_pad_batch(prompts: list[list[int]], device) -> tuple[torch.Tensor, ...]:
    """Left-pad with END / position (0,0,0) and build the bool mask (src/inference.py:877-890)."""
    n = max(len(p) for p in prompts)
    B = len(prompts)
    ids = np.full((B, n), END_TOKEN_ID, dtype=np.int64)
    pos = np.zeros((B, n, 3), dtype=np.int64)
    mask = np.zeros((B, n), dtype=bool)
    for i, p in enumerate(prompts):
        k = len(p)
        ids[i, n - k:] = p
        pos[i, n - k:] = compute_positions_3d(p)
        mask[i, n - k:] = True
    to = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    return to(ids), to(pos), to(mask)


def predict_with_augmentations(model: TinyTransformer, task: dict, test_idx: int, device,
                               example_id: int = 0, use_train_examples: bool = True,
                               num_color_perms: int = 8, max_output_tokens: int = 900,
                               num_samples: int = 1, sample_temperature: float = 0.0,
                               sample_top_k: int | None = None, constrain_decoding: bool = False,
                               palette_penalty: float = 2.0, shape_penalty: float = 2.0,
                               batched: bool = True, use_compile: bool = False,
                               max_batch_size: int = 16, fuse_chunks: bool = True):
    """All dihedral x colour-permutation predictions for AAIVR voting
    (src/inference.py:697-920): list of (grid | None, dihedral_idx, perm_tuple | None).

    The reference runs the prompts in left-padded chunks of ``max_batch_size`` (16) when
    ``batched``, otherwise one prompt at a time; the chunking is part of its results (each
    chunk's padding fixes its ``lengths-1`` rows, and a chunk stops when all of its rows have
    emitted END).  With greedy decoding and ``fuse_chunks`` (the default) every chunk runs in
    ONE batch with those semantics kept per row (``_predict_fused``); sampling, whose random
    draws depend on the batch, keeps the chunk loop, as does ``fuse_chunks=False``."""
    del use_compile
    num_samples = max(1, num_samples)
    base_palette = _collect_palette(task, test_idx) if constrain_decoding else None
    base_shape = _infer_output_shape(task) if constrain_decoding else None
    return _predict_augmentations(model, task, test_idx, device, example_id, use_train_examples,
                                  num_color_perms, max_output_tokens, num_samples,
                                  sample_temperature, sample_top_k, constrain_decoding,
                                  base_palette, base_shape, palette_penalty, shape_penalty,
                                  batched, max_batch_size, fuse_chunks)


def _predict_augmentations(model, task, test_idx, device, example_id, use_train_examples,
                           num_color_perms, max_output_tokens, num_samples, sample_temperature,
                           sample_top_k, constrain_decoding, base_palette, base_shape,
                           palette_penalty, shape_penalty, batched, max_batch_size,
                           fuse_chunks=True):
    """The body of predict_with_augmentations after its palette / shape inference: the
    reference's batched (chunks of ``max_batch_size``) or sequential loop."""
    model.eval()
    num_samples = max(1, num_samples)
    chunk = max_batch_size if batched else 1
    fused = fuse_chunks and sample_temperature <= 0 and 8 * num_color_perms * num_samples > 1
    grids = (_task_grids(task, test_idx, use_train_examples)
             if fused and DEVICE_PROMPTS else None)
    variants = _build_variants(task, test_idx, use_train_examples, num_color_perms, num_samples,
                               constrain_decoding, base_palette, base_shape,
                               tokenize=grids is None)
    if fused:
        return _predict_fused(model, variants, chunk, device, example_id, max_output_tokens,
                              constrain_decoding, palette_penalty, shape_penalty, grids,
                              num_color_perms)
    preds = []
    for c0 in range(0, len(variants), chunk):
        part = variants[c0:c0 + chunk]
        constraints = None
        if constrain_decoding:
            constraints = _chunk_constraints(part, device, palette_penalty, shape_penalty,
                                             batched)
        if batched:
            ids, pos, mask = left_pad_batch([v.tokens for v in part], device)
        else:
            ids, pos, mask = left_pad_batch([part[0].tokens], device)
            mask = None
        ex = torch.full((len(part),), example_id, dtype=torch.long, device=device)
        with torch.no_grad():
            out_ids = generate_output(model, ids, pos, ex, attention_mask=mask,
                                      max_new_tokens=max_output_tokens,
                                      temperature=sample_temperature, top_k=sample_top_k,
                                      stop_on_end=True, constraints=constraints)
        rows = out_ids.cpu().tolist()
        for v, seq in zip(part, rows):
            seps = [j for j, t in enumerate(seq) if t == IO_SEP_TOKEN_ID]
            grid = decode_output_grid(seq[seps[-1]:]) if seps else None
            preds.append((grid, v.dihedral, v.perm))
    return preds


def _predict_fused(model: TinyTransformer, variants: list[_Variant], chunk: int, device,
                   example_id: int, max_output_tokens: int, constrain: bool,
                   palette_penalty: float, shape_penalty: float, grids: list | None = None,
                   num_color_perms: int = 0):
    """Greedy predictions of every variant from one generation over all of them, equal to the
    reference's loop over left-padded chunks of ``chunk`` rows (src/inference.py:829-918).

    Row i of chunk c (padded there to width L_c, here to the batch-wide S):
    * its prefill logits and initial grid state come from the reference's index lengths-1 in its
      chunk, i.e. index S - L_c + lengths-1 here (``mdl_grid_init`` row_shift; the extra left
      pads are END tokens at (0, 0, 0) whose hidden states equal the chunk's own pads);
    * it keeps the first g_c generated tokens, where the chunk's budget is
      b_c = min(L_c + max_output_tokens, max_seq_len) - L_c and g_c = min(b_c, 1 + the latest
      first-END index over the chunk's rows), b_c if a row never emits END: the reference stops
      a chunk once all of its rows have emitted END, and keeps what finished rows produced until
      then;
    * greedy rows never interact (attention, norms and the argmax are per row; constraints are
      per row), so the tokens themselves do not depend on the batch.
    The one generation runs until every row has emitted END or the largest budget is spent, so
    every row has at least its g_c tokens.

    With ``grids`` (the task's rectangular grids) the prompts are built on the device
    (``mdl_build_prompts``); otherwise from the variants' host tokens.  Every prompt ends with
    IO_SEP, so a row's grid is decoded from its generated tokens alone."""
    cfg = model.config
    n = len(variants)
    if grids is not None:
        ids, pos, mask, lens = _device_prompts(grids, variants, num_color_perms, device)
    else:
        lens = [len(v.tokens) for v in variants]
        ids, pos, mask = left_pad_batch([v.tokens for v in variants], device)
    widths = [max(lens[c0:c0 + chunk]) for c0 in range(0, n, chunk)]
    budgets = [min(w + max_output_tokens, cfg.max_seq_len) - w for w in widths]
    S = ids.shape[1]
    gen_max = max(budgets)
    gen = torch.empty(n, 0, dtype=torch.int64)
    fin = torch.full((n,), -1, dtype=torch.int32)
    if gen_max > 0:
        shift = torch.tensor([S - widths[i // chunk] for i in range(n)], dtype=torch.int32)
        constraints = (_chunk_constraints(variants, device, palette_penalty, shape_penalty, True)
                       if constrain else None)
        ex = torch.full((n,), example_id, dtype=torch.long, device=device)
        with torch.no_grad():
            out_ids, finish, _ = _generate(model, ids, pos, ex, mask, S + gen_max, 0.0, None, True,
                                           constraints, row_shift=shift)
        gen = out_ids[:, S:].cpu()
        fin = finish.cpu()
    preds = []
    for c, c0 in enumerate(range(0, n, chunk)):
        rows = range(c0, min(c0 + chunk, n))
        f = fin[c0:c0 + chunk]
        g = budgets[c]
        if g > 0 and bool((f >= 0).all()):
            g = min(g, int(f.max()) + 1)
        for i in rows:
            seq = [IO_SEP_TOKEN_ID] + gen[i, :max(g, 0)].tolist()   # the prompt's last token on
            seps = [j for j, t in enumerate(seq) if t == IO_SEP_TOKEN_ID]
            preds.append((decode_output_grid(seq[seps[-1]:]), variants[i].dihedral,
                          variants[i].perm))
    return preds


def _chunk_constraints(part: list[_Variant], device, palette_penalty, shape_penalty,
                       batched: bool) -> DecodingConstraints:
    """Per-row palette / target-shape tensors of one chunk (src/inference.py:842-875 batched,
    :973-992 sequential)."""
    n = len(part)
    pal = None
    if batched:
        m = torch.ones(n, 10, dtype=torch.bool)
        any_pal = False
        for i, v in enumerate(part):
            if v.palette:
                any_pal = True
                m[i] = False
                for c in v.palette:
                    if 0 <= c < 10:
                        m[i, c] = True
        pal = m.to(device) if any_pal else None
    elif part[0].palette:
        m = torch.zeros(1, 10, dtype=torch.bool)
        for c in part[0].palette:
            if 0 <= c < 10:
                m[0, c] = True
        pal = m.to(device)
    shp = torch.full((n, 2), -1, dtype=torch.long)
    any_shape = False
    for i, v in enumerate(part):
        if v.shape is not None:
            any_shape = True
            shp[i] = torch.tensor(v.shape)
    return DecodingConstraints(palette_mask=pal, target_shape=shp.to(device) if any_shape else None,
                               palette_penalty=palette_penalty, shape_penalty=shape_penalty)


# =============================================================================================
# the reference's module-level helpers, for code that calls or patches them
# (src/inference.py:285-479, :763-1003); the generation path itself does not go through them
# =============================================================================================

def _apply_logit_constraints(logits: torch.Tensor, grid_state,
                             constraints: DecodingConstraints | None) -> torch.Tensor:
    """src/inference.py:285-364 with the reference's arguments: logits [B, V] or [B, 1, V],
    changed in place and returned; ``grid_state`` is the state after the current token (any
    object with the ``x`` / ``y`` tensors of GridStateUpdater)."""
    if constraints is None:
        return logits
    apply_logit_constraints(logits.view(-1, logits.shape[-1]), grid_state.x, grid_state.y,
                            constraints)
    return logits


def _build_sdpa_mask(attention_mask: torch.Tensor | None, dtype: torch.dtype):
    """src/inference.py:372-380: a [B, S] bool mask as the additive [B, 1, 1, S] SDPA mask
    (0 where True, -inf where False) in ``dtype``; None stays None."""
    if attention_mask is None:
        return None
    keep = attention_mask.bool()[:, None, None, :]
    return torch.zeros(keep.shape, dtype=dtype, device=keep.device).masked_fill(~keep,
                                                                                float("-inf"))


def _prefill(model: TinyTransformer, input_ids: torch.Tensor, positions_3d: torch.Tensor,
             example_ids: torch.Tensor | None, cache: StaticKVCache,
             attention_mask: torch.Tensor | None = None) -> torch.Tensor:
    """src/inference.py:383-424 on the HIP kernels: every layer over the [B, S] prompt, K / V
    into slots [0, S) of ``cache`` (a StaticKVCache of this module, in the model's dtype, not yet
    advanced), then cache.advance(S).  Returns the logits [B, 1, V] (model dtype) of row
    lengths-1 of each row -- the reference's index on left-padded batches -- or of the last
    column without a mask."""
    eng = engine_for(model)
    dev = eng._check_device(input_ids)
    cfg = model.config
    B, S = input_ids.shape
    if cache.seq_len != 0:
        raise ValueError("_prefill writes cache slots [0, S): pass a cache that is not advanced")
    ids = input_ids.to(torch.int64).contiguous()
    pos = positions_3d.to(device=dev, dtype=torch.int64).contiguous()
    ex = None if example_ids is None else example_ids.to(device=dev,
                                                          dtype=torch.int64).contiguous()
    eng._validate_ids(ids, ex)
    with torch.no_grad():
        W = eng.packed(dev)
        want = torch.float32 if W.f32 else torch.bfloat16
        if cache.cache.dtype != want:
            raise TypeError(f"the cache must be {want} for this model (got {cache.cache.dtype})")
        mask, kv_start = eng.key_mask_and_start(attention_mask, dev, S)
        sc = Scratch.for_prompt(B * S, cfg, dev, W.f32)
        eng.run_prompt(W, ids, pos, ex, mask, kv_start, True, cache.layer, sc)
        if attention_mask is None:
            last = torch.full((B,), S - 1, dtype=torch.int64, device=dev)
        else:
            last = (attention_mask.to(dev).long().sum(1) - 1).clamp(min=0)
        rows = (torch.arange(B, device=dev) * S + last).to(torch.int32)
        logits = torch.empty(B, cfg.vocab_size, dtype=torch.float32, device=dev)
        K.lm_head(sc.x, rows, B, W.ln_f, W.eps, W.head, logits, None,
                  x_tiled=sc.fused or sc.tiled)
    cache.advance(S)
    return logits.to(model.lm_head.weight.dtype)[:, None]


def _decode_step(model: TinyTransformer, token: torch.Tensor, position: torch.Tensor,
                 example_ids: torch.Tensor | None, cache: StaticKVCache,
                 attention_mask: torch.Tensor | None = None) -> torch.Tensor:
    """src/inference.py:427-459 on the HIP kernels, host-launched: the token [B, 1] at position
    [B, 1, 3] through every layer, its K / V into slot cache.seq_len, attention over slots
    [0, seq_len] where ``attention_mask`` ([B, >= seq_len + 1] bool, may be None) allows, then
    cache.advance(1).  Returns the logits [B, 1, V] (model dtype)."""
    eng = engine_for(model)
    dev = eng._check_device(token)
    cfg = model.config
    B = token.shape[0]
    H = cfg.n_heads
    t = cache.seq_len
    if not 0 <= t < cache.max_seq_len:
        raise ValueError("the cache is full")
    tok = token.reshape(B).to(device=dev, dtype=torch.int64).contiguous()
    ex = (torch.zeros(B, dtype=torch.int64, device=dev) if example_ids is None
          else example_ids.to(device=dev, dtype=torch.int64).contiguous())
    eng._validate_ids(tok, ex)
    gen = Generator(model)
    f32 = model_form(model) == "fp32"
    with torch.no_grad():
        W = eng.packed(dev)
        want = torch.float32 if W.f32 else torch.bfloat16
        if cache.cache.dtype != want:
            raise TypeError(f"the cache must be {want} for this model (got {cache.cache.dtype})")
        pmask = None
        if attention_mask is not None:
            pmask = attention_mask[:, :t + 1].to(device=dev, dtype=torch.uint8).contiguous()
        slots = cache.max_seq_len
        split = choose_split_len(B * H, slots)
        nbytes = K.attn_decode_workspace_bytes(B, H, slots, split)
        i32 = lambda: torch.zeros(B, dtype=torch.int32, device=dev)  # noqa: E731
        st = DecodeState(
            B=B, S=0 if pmask is None else pmask.shape[1], total=slots, ex=ex, pmask=pmask,
            kv_start=None, last_row=i32(), holes=None, order=None, gx=i32(), gy=i32(),
            gio=torch.zeros(B, dtype=torch.uint8, device=dev),
            pos=position.reshape(B, 3).to(device=dev, dtype=torch.int64).contiguous(), tok=tok,
            counters=torch.tensor([t, 0], dtype=torch.int32, device=dev),
            out_ids=torch.empty(B, 0, dtype=torch.int64, device=dev),
            finish=i32(), logits=torch.empty(B, cfg.vocab_size, dtype=torch.float32, device=dev),
            cache=cache,
            ws=(torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=dev)
                if nbytes else None),
            sc=Scratch.alloc(B, cfg.d_model, cfg.d_ff, dev, f32=f32,
                             tiled=DECODE_TILED and tiles_supported(cfg.d_model, cfg.d_ff)),
            split_len=split)
        gen.decode_layers(st, W, want_logits=True)
    cache.advance(1)
    return st.logits.to(model.lm_head.weight.dtype)[:, None]


def _get_decode_fn(use_compile: bool):
    """src/inference.py:462-479: the decode-step function.  There is no compiler on this path,
    so ``use_compile`` selects nothing; generate_output replays a captured HIP graph of its own
    step instead."""
    del use_compile
    return _decode_step


def _predict_augmentations_batched(model, task, test_idx, device, example_id,
                                   use_train_examples, num_color_perms, max_output_tokens,
                                   num_samples, sample_temperature, sample_top_k,
                                   constrain_decoding, base_palette, base_shape, palette_penalty,
                                   shape_penalty, use_compile, max_batch_size: int = 16):
    """src/inference.py:763-920: the augmentations in left-padded chunks of max_batch_size."""
    del use_compile
    return _predict_augmentations(model, task, test_idx, device, example_id, use_train_examples,
                                  num_color_perms, max_output_tokens, num_samples,
                                  sample_temperature, sample_top_k, constrain_decoding,
                                  base_palette, base_shape, palette_penalty, shape_penalty, True,
                                  max_batch_size)


def _predict_augmentations_sequential(model, task, test_idx, device, example_id,
                                      use_train_examples, num_color_perms, max_output_tokens,
                                      num_samples, sample_temperature, sample_top_k,
                                      constrain_decoding, base_palette, base_shape,
                                      palette_penalty, shape_penalty, use_compile):
    """src/inference.py:923-1003: one augmentation at a time (no padding, no mask)."""
    del use_compile
    return _predict_augmentations(model, task, test_idx, device, example_id, use_train_examples,
                                  num_color_perms, max_output_tokens, num_samples,
                                  sample_temperature, sample_top_k, constrain_decoding,
                                  base_palette, base_shape, palette_penalty, shape_penalty, False,
                                  1)
