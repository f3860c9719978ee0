"""CPU restatement of the TinyTransformer inference path -- test infrastructure only.

Only tests, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg use this module; the
product (``mdlarc_scale_amd``) never imports it.  Everything runs in torch on the CPU in the dtype
the caller picks (fp32 is "the fp32 CPU reference"; fp64 is used by closed-form checks).

Each function names the reference lines it restates.  Reference = shyampathak22/mdlARC_scale.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

VOCAB_SIZE = 14
START, NEWLINE, IO_SEP, END = 10, 11, 12, 13


@dataclass
class OracleConfig:
    """Shape fields of ``TransformerConfig`` (src/transformer.py:15-34) that the path reads."""

    d_model: int
    n_heads: int
    n_layers: int
    d_ff: int
    num_examples: int = 1280
    max_seq_len: int = 1863
    max_x: int = 32
    max_y: int = 32
    max_z: int = 8
    rope_base: float = 10000.0
    norm_eps: float = 1e-5
    use_example_embedding: bool = True
    vocab_size: int = VOCAB_SIZE

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads


# --------------------------------------------------------------------------------------------
# elementary ops
# --------------------------------------------------------------------------------------------

def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``RMSNorm.forward`` (src/transformer.py:45-48): x * rsqrt(mean(x^2) + eps) * weight."""
    ms = (x * x).mean(dim=-1, keepdim=True)
    return x * torch.rsqrt(ms + eps) * weight


def rope3d_split(head_dim: int) -> tuple[int, int, int]:
    """Pairs per axis (src/transformer.py:87-90): x and y get n//3 pairs, z the remainder."""
    n = head_dim // 2
    return n // 3, n // 3, n - 2 * (n // 3)


def rope3d_tables(cfg: OracleConfig) -> dict[str, torch.Tensor]:
    """cos/sin tables per axis, built in fp32 as ``_build_cache``/``_make_inv_freq`` do
    (src/transformer.py:95-126): inv_freq_j = 1 / base^(2j / (2p)), angle = pos * inv_freq."""
    px, py, pz = rope3d_split(cfg.head_dim)
    out = {}
    for axis, pairs, npos in (("x", px, cfg.max_x), ("y", py, cfg.max_y), ("z", pz, cfg.max_z)):
        dim = 2 * pairs
        inv = 1.0 / (cfg.rope_base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
        ang = torch.outer(torch.arange(npos, dtype=torch.float32), inv)
        out["cos_" + axis] = ang.cos()
        out["sin_" + axis] = ang.sin()
    return out


def apply_rope3d(t: torch.Tensor, pos: torch.Tensor, tables: dict[str, torch.Tensor],
                 cfg: OracleConfig) -> torch.Tensor:
    """Rotate interleaved pairs of ``t`` [..., S, H, hd] by 3D position ``pos`` [..., S, 3].

    ``RotaryEmbedding3D.apply_rotary`` (src/transformer.py:132-187) with ``_rotate_half``
    (:51-58): coordinates are clamped to [0, max-1] (:152-154); pair j of the head uses the x table
    for j < px, y for px <= j < px+py, z otherwise (:167-177); (a, b) -> (a c - b s, b c + a s).
    """
    xp = pos[..., 0].clamp(0, cfg.max_x - 1).long()
    yp = pos[..., 1].clamp(0, cfg.max_y - 1).long()
    zp = pos[..., 2].clamp(0, cfg.max_z - 1).long()
    dt = t.dtype
    cos = torch.cat([tables["cos_x"][xp], tables["cos_y"][yp], tables["cos_z"][zp]], -1).to(dt)
    sin = torch.cat([tables["sin_x"][xp], tables["sin_y"][yp], tables["sin_z"][zp]], -1).to(dt)
    cos, sin = cos.unsqueeze(-2), sin.unsqueeze(-2)          # broadcast over heads
    a, b = t[..., 0::2], t[..., 1::2]
    ra = a * cos - b * sin
    rb = b * cos + a * sin
    return torch.stack((ra, rb), dim=-1).flatten(-2)


def silu(a: torch.Tensor) -> torch.Tensor:
    """``F.silu`` as used by ``FeedForward`` (src/transformer.py:447): a * sigmoid(a)."""
    return a * torch.sigmoid(a)


def swiglu_ffn(x: torch.Tensor, w: dict[str, torch.Tensor], p: str) -> torch.Tensor:
    """``FeedForward.forward`` (src/transformer.py:446-451), dropout = identity in eval:
    fc_down(silu(fc_gate(x)) * fc_up(x)), every Linear with its bias (:441-443)."""
    g = x @ w[p + "fc_gate.weight"].T + w[p + "fc_gate.bias"]
    u = x @ w[p + "fc_up.weight"].T + w[p + "fc_up.bias"]
    return (silu(g) * u) @ w[p + "fc_down.weight"].T + w[p + "fc_down.bias"]


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, key_mask: torch.Tensor | None,
              causal: bool, q_offset: int = 0) -> torch.Tensor:
    """softmax(q k^T / sqrt(hd) + mask) v with fully-masked rows -> 0.

    Restates ``F.scaled_dot_product_attention`` at src/inference.py:409 (prefill: float key mask
    from ``_build_sdpa_mask`` :372-380 AND top-left causal) and :452 (decode: key mask only).
    q [B,H,Sq,hd], k/v [B,H,Sk,hd], key_mask [B,Sk] bool (True = attend).  Query i may see key j
    iff key_mask[b, j] and (not causal or j <= i + q_offset).  A query with no visible key
    returns zeros (what torch's CPU SDPA returns for an all -inf row).
    """
    B, H, Sq, hd = q.shape
    Sk = k.shape[2]
    allowed = torch.ones(B, 1, Sq, Sk, dtype=torch.bool)
    if key_mask is not None:
        allowed = allowed & key_mask.bool()[:, None, None, :]
    if causal:
        i = torch.arange(Sq)[:, None] + q_offset
        j = torch.arange(Sk)[None, :]
        allowed = allowed & (j <= i)[None, None]
    s = (q @ k.transpose(-1, -2)) * (1.0 / math.sqrt(hd))
    s = s.masked_fill(~allowed, float("-inf"))
    m = s.amax(dim=-1, keepdim=True)
    any_ok = allowed.any(dim=-1, keepdim=True)
    m = torch.where(any_ok, m, torch.zeros_like(m))
    p = torch.exp(s - m)                       # exp(-inf) = 0 on masked keys
    den = p.sum(dim=-1, keepdim=True)
    o = (p @ v) / torch.where(any_ok, den, torch.ones_like(den))
    return torch.where(any_ok, o, torch.zeros_like(o))


# --------------------------------------------------------------------------------------------
# model
# --------------------------------------------------------------------------------------------

class OracleModel:
    """Weights (reference ``state_dict`` keys, src/transformer.py:523-545) in one CPU dtype."""

    def __init__(self, cfg: OracleConfig, state: dict[str, torch.Tensor],
                 dtype: torch.dtype = torch.float32):
        self.cfg = cfg
        self.dtype = dtype
        self.w = {k: torch.as_tensor(v).detach().to("cpu", dtype) for k, v in state.items()}
        self.tables = rope3d_tables(cfg)

    # -- embedding -----------------------------------------------------------------------
    def embed(self, ids: torch.Tensor, ex_ids: torch.Tensor | None) -> torch.Tensor:
        """Token + broadcast example embedding (src/transformer.py:584-589,
        src/inference.py:393-395 and :433-435)."""
        x = self.w["token_embed.weight"][ids]
        if ex_ids is not None and self.cfg.use_example_embedding:
            x = x + self.w["example_embed.weight"][ex_ids].unsqueeze(1)
        return x

    def _qkv(self, x: torch.Tensor, li: int, pos: torch.Tensor):
        """ln1 -> qkv_proj -> split [B,S,3,H,hd] -> RoPE on q,k (src/inference.py:401-404)."""
        c, w, p = self.cfg, self.w, f"blocks.{li}."
        B, S, _ = x.shape
        h = rmsnorm(x, w[p + "ln1.weight"], c.norm_eps)
        qkv = (h @ w[p + "attn.qkv_proj.weight"].T).reshape(B, S, 3, c.n_heads, c.head_dim)
        q, k, v = qkv.unbind(2)
        q = apply_rope3d(q, pos, self.tables, c)
        k = apply_rope3d(k, pos, self.tables, c)
        return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)

    def _finish_block(self, x: torch.Tensor, o: torch.Tensor, li: int) -> torch.Tensor:
        """out_proj + residual, then ln2 -> SwiGLU + residual (src/inference.py:410-413)."""
        w, p = self.w, f"blocks.{li}."
        B, H, S, hd = o.shape
        x = x + o.transpose(1, 2).reshape(B, S, H * hd) @ w[p + "attn.out_proj.weight"].T
        return x + swiglu_ffn(rmsnorm(x, w[p + "ln2.weight"], self.cfg.norm_eps), w, p + "ffn.")

    def head(self, x: torch.Tensor) -> torch.Tensor:
        """ln_f -> lm_head (src/transformer.py:596-597)."""
        return rmsnorm(x, self.w["ln_f.weight"], self.cfg.norm_eps) @ self.w["lm_head.weight"].T

    def forward(self, ids: torch.Tensor, pos: torch.Tensor, ex_ids: torch.Tensor | None = None,
                attention_mask: torch.Tensor | None = None, is_causal: bool = True) -> torch.Tensor:
        """``TinyTransformer.forward`` (src/transformer.py:562-599) -> logits [B,S,V]."""
        x = self.embed(ids, ex_ids)
        for li in range(self.cfg.n_layers):
            q, k, v = self._qkv(x, li, pos)
            o = attention(q, k, v, attention_mask, causal=is_causal)
            x = self._finish_block(x, o, li)
        return self.head(x)

    # -- static-cache inference ---------------------------------------------------------------
    def new_cache(self, batch: int, slots: int) -> torch.Tensor:
        """``StaticKVCache`` storage (src/inference.py:73-77): zeros [N_L, 2, B, H, slots, hd]."""
        c = self.cfg
        return torch.zeros(c.n_layers, 2, batch, c.n_heads, slots, c.head_dim, dtype=self.dtype)

    def prefill(self, ids: torch.Tensor, pos: torch.Tensor, ex_ids: torch.Tensor | None,
                cache: torch.Tensor, attention_mask: torch.Tensor | None) -> torch.Tensor:
        """``_prefill`` (src/inference.py:383-424): fill slots [0, S) and return logits [B,V] of
        row ``lengths-1`` (the right-padding index the reference applies to its left-padded
        batches, :420-424), or of the last column when there is no mask (:417-418)."""
        B, S = ids.shape
        x = self.embed(ids, ex_ids)
        for li in range(self.cfg.n_layers):
            q, k, v = self._qkv(x, li, pos)
            cache[li, 0, :, :, :S] = k
            cache[li, 1, :, :, :S] = v
            o = attention(q, k, v, attention_mask, causal=True)
            x = self._finish_block(x, o, li)
        if attention_mask is None:
            return self.head(x[:, -1])
        last = (attention_mask.long().sum(1) - 1).clamp(min=0)
        return self.head(x[torch.arange(B), last])

    def decode_step(self, token: torch.Tensor, position: torch.Tensor,
                    ex_ids: torch.Tensor | None, cache: torch.Tensor, seq_len: int,
                    key_mask: torch.Tensor | None) -> torch.Tensor:
        """``_decode_step`` (src/inference.py:427-459): one token per row, K/V written at slot
        ``seq_len``, attention over slots [0, seq_len] with ``key_mask`` [B, seq_len+1]."""
        x = self.embed(token.view(-1, 1), ex_ids)
        n = seq_len + 1
        for li in range(self.cfg.n_layers):
            q, k, v = self._qkv(x, li, position.view(-1, 1, 3))
            cache[li, 0, :, :, seq_len] = k[:, :, 0]
            cache[li, 1, :, :, seq_len] = v[:, :, 0]
            o = attention(q, cache[li, 0, :, :, :n], cache[li, 1, :, :, :n], key_mask,
                          causal=False)
            x = self._finish_block(x, o, li)
        return self.head(x[:, 0])


# --------------------------------------------------------------------------------------------
# grid-state position tracking
# --------------------------------------------------------------------------------------------

class GridState:
    """``GridStateUpdater`` (src/inference.py:104-168): per-row (x, y, in_output) that yields the
    3D position of each generated token.  Defaults max_x=30, max_y=29 (:107)."""

    def __init__(self, x: torch.Tensor, y: torch.Tensor, in_output: torch.Tensor,
                 max_x: int = 30, max_y: int = 29):
        self.x, self.y = x.long().clone(), y.long().clone()
        self.in_output = in_output.bool().clone()
        self.max_x, self.max_y = max_x, max_y

    def update(self, tok: torch.Tensor) -> torch.Tensor:
        """Position of ``tok`` [B] from the current state, then advance the state (:127-168)."""
        tok = tok.view(-1).long()
        st, sp, en, nl = tok == START, tok == IO_SEP, tok == END, tok == NEWLINE
        color = tok < 10
        z = torch.where(self.in_output, 3, 1)
        z = torch.where(st, 0, z)
        z = torch.where(sp, 2, z)
        z = torch.where(en, 4, z)
        px = torch.where(st | sp | en | nl, 0, self.x.clamp(0, self.max_x))
        py = torch.where(st | sp | en, 0, self.y.clamp(0, self.max_y))
        out = torch.stack([px, py, z], -1)

        x = torch.where(st | sp, 0, self.x)
        y = torch.where(st | sp, 0, self.y)
        io = torch.where(st, False, self.in_output)
        io = torch.where(sp, True, io)
        x = torch.where(nl, 0, x)
        y = torch.where(nl, (y + 1).clamp(max=self.max_y), y)
        x = torch.where(color, (x + 1).clamp(max=self.max_x), x)
        self.x, self.y, self.in_output = x.clamp(0, self.max_x), y.clamp(0, self.max_y), io
        return out


def derive_initial_state(ids: torch.Tensor, pos: torch.Tensor, mask: torch.Tensor | None,
                         max_x: int = 30, max_y: int = 29):
    """``_derive_initial_state_from_prompt`` (src/inference.py:171-221): grid state after the
    prompt, read from the token at index ``lengths-1`` (same right-pad index as ``_prefill``)."""
    B, S = ids.shape
    mask = torch.ones(B, S, dtype=torch.bool) if mask is None else mask.bool()
    n = mask.long().sum(1)
    last = (n - 1).clamp(min=0)
    r = torch.arange(B)
    tok, lp = ids[r, last], pos[r, last]
    st, sp, nl = tok == START, tok == IO_SEP, tok == NEWLINE
    io = torch.where(st, False, lp[:, 2] >= 3)
    io = torch.where(sp, True, io)
    x = torch.where(st | sp, 0, lp[:, 0])
    y = torch.where(st | sp, 0, lp[:, 1])
    x = torch.where(nl, 0, x)
    y = torch.where(nl, (y + 1).clamp(max=max_y), y)
    x = torch.where(tok < 10, (x + 1).clamp(max=max_x), x)
    x, y = x.clamp(0, max_x), y.clamp(0, max_y)
    has = n > 0
    return torch.where(has, x, 0), torch.where(has, y, 0), torch.where(has, io, True)


# --------------------------------------------------------------------------------------------
# decoding constraints
# --------------------------------------------------------------------------------------------

@dataclass(frozen=True)
class OracleConstraints:
    """Fields of ``DecodingConstraints`` (src/inference.py:36-43), same defaults."""

    palette_mask: torch.Tensor | None = None     # bool [B or 1, 10]
    target_shape: torch.Tensor | None = None     # long [B or 1, 2]; -1 = no shape
    palette_penalty: float = 2.0
    shape_penalty: float = 2.0
    disallow_tokens: tuple[int, ...] = (START, IO_SEP)


def _rows_of(t: torch.Tensor, batch: int, width: int) -> torch.Tensor | None:
    """A constraint tensor as [batch, width]: reshaped to 2D, a single row broadcast, any other
    batch mismatch -> None (the constraint is then skipped) (src/inference.py:305-311, :316-322)."""
    if t.dim() != 2:
        t = t.reshape(-1, t.shape[-1] if width == 10 else 2)
    if t.shape[0] != batch:
        return t.expand(batch, -1) if t.shape[0] == 1 else None
    return t


def apply_logit_constraints(logits: torch.Tensor, gx: torch.Tensor, gy: torch.Tensor,
                            c: OracleConstraints | None) -> torch.Tensor:
    """``_apply_logit_constraints`` (src/inference.py:285-364) on logits [B, V] (the reference's
    [B, 1, V] without the middle axis), in place; (gx, gy) is the grid state after the current
    token.  Order and rounding as the reference: disallowed tokens -> -inf (:296-297); colours
    0-9 minus palette_penalty * (not allowed) (:299-312); with a target shape (h, w >= 0):
    colours minus shape_penalty * (x >= w) (:347-350), NEWLINE minus shape_penalty * (x < w)
    (:351-353), then colours and NEWLINE each minus shape_penalty * (y >= h) (:354-357), every
    penalty a separate fp32 subtraction of (indicator * penalty).  A grid-state batch that
    neither equals nor broadcasts the shape batch ends the rule early (:337-343)."""
    if c is None:
        return logits
    B = logits.shape[0]
    for tok in c.disallow_tokens:
        logits[:, tok] = float("-inf")
    if c.palette_mask is not None:
        pm = _rows_of(c.palette_mask, B, 10)
        if pm is not None:
            logits[:, :10] = logits[:, :10] - (~pm).to(logits.dtype) * c.palette_penalty
    if c.target_shape is not None:
        ts = _rows_of(c.target_shape, B, 2)
        if ts is not None:
            th, tw = ts[:, 0].contiguous().view(-1), ts[:, 1].contiguous().view(-1)
            has = (th >= 0) & (tw >= 0)
            if bool(has.any()):
                x, y = gx.contiguous().view(-1), gy.contiguous().view(-1)
                if x.shape[0] != tw.shape[0]:
                    if tw.shape[0] != 1:
                        return logits
                    th, tw, has = th.expand(x.shape[0]), tw.expand(x.shape[0]), has.expand(
                        x.shape[0])
                full, open_, past = has & (x >= tw), has & (x < tw), has & (y >= th)
                pen = c.shape_penalty
                if bool(full.any()):
                    logits[:, :10] = logits[:, :10] - full.to(logits.dtype)[:, None] * pen
                if bool(open_.any()):
                    logits[:, NEWLINE] = logits[:, NEWLINE] - open_.to(logits.dtype) * pen
                if bool(past.any()):
                    p = past.to(logits.dtype) * pen
                    logits[:, :10] = logits[:, :10] - p[:, None]
                    logits[:, NEWLINE] = logits[:, NEWLINE] - p
    return logits


# --------------------------------------------------------------------------------------------
# batched greedy generation
# --------------------------------------------------------------------------------------------

@dataclass
class GenerateTrace:
    tokens: torch.Tensor                 # [B, S + g]
    step_logits: list[torch.Tensor]      # g entries of [B, V]; entry 0 from the prefill
    step_positions: list[torch.Tensor]   # g-1 entries of [B, 3] fed to the decode steps
    raw_logits: list[torch.Tensor] = None  # g entries of [B, V] before the constraints


def generate_output(model: OracleModel, ids: torch.Tensor, pos: torch.Tensor,
                    ex_ids: torch.Tensor | None = None,
                    attention_mask: torch.Tensor | None = None, max_new_tokens: int = 900,
                    stop_on_end: bool = True,
                    constraints: OracleConstraints | None = None) -> GenerateTrace:
    """Greedy ``generate_output`` (src/inference.py:487-628), temperature <= 0.

    Bug-compatible with the reference: example ids default to zeros (:524-525); the total length
    is capped at ``max_seq_len`` and an over-long prompt is returned unchanged (:534-537); the
    first token and the initial grid state come from index ``lengths-1``; rows that emitted END
    keep generating; the loop breaks before a step once every row has emitted END (:593-595);
    argmax takes the first index on ties (:573-574, :610-611).  ``constraints`` are applied
    before every argmax (:572, :609), with the grid state after the prompt for the first token
    and after the previous token for the others; ``step_logits`` holds the constrained logits.
    """
    B, S = ids.shape
    if ex_ids is None:
        ex_ids = torch.zeros(B, dtype=torch.long)
    prompt_mask = (torch.ones(B, S, dtype=torch.bool) if attention_mask is None
                   else attention_mask.bool())
    total = min(S + max_new_tokens, model.cfg.max_seq_len)
    max_new = total - S
    if max_new <= 0:
        return GenerateTrace(ids.clone(), [], [], [])
    cache = model.new_cache(B, total)
    gx, gy, gio = derive_initial_state(ids, pos, prompt_mask)
    grid = GridState(gx, gy, gio)
    full_mask = torch.zeros(B, total, dtype=torch.bool)
    full_mask[:, :S] = prompt_mask

    logits = model.prefill(ids, pos, ex_ids, cache, prompt_mask)
    raw = [logits.clone()]
    logits = apply_logit_constraints(logits, grid.x, grid.y, constraints)
    nxt = logits.argmax(-1)
    out, lg, ps = [ids, nxt[:, None]], [logits], []
    finished = (nxt == END) if stop_on_end else torch.zeros(B, dtype=torch.bool)
    full_mask[:, S] = True
    for step in range(1, max_new):
        if stop_on_end and bool(finished.all()):
            break
        p = grid.update(nxt)
        ps.append(p)
        seq = S + step - 1
        logits = model.decode_step(nxt, p, ex_ids, cache, seq, full_mask[:, :seq + 1])
        raw.append(logits.clone())
        logits = apply_logit_constraints(logits, grid.x, grid.y, constraints)
        nxt = logits.argmax(-1)
        lg.append(logits)
        if stop_on_end:
            finished = finished | (nxt == END)
        out.append(nxt[:, None])
        full_mask[:, S + step] = True
    return GenerateTrace(torch.cat(out, 1), lg, ps, raw)
