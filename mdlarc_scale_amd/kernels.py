"""Tensor-level wrappers of the C-ABI entry points.

Each wrapper checks device, dtype, shape and contiguity of its torch tensors, then passes raw
device pointers and the current HIP stream to the library.  Checks that need no device data run
here, in Python, before any launch (the C side repeats the ones it can see); a failed check or a
non-zero library status raises ``RuntimeError`` / ``ValueError``.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

BF16, F32, I64, I32, U8 = torch.bfloat16, torch.float32, torch.int64, torch.int32, torch.uint8
HEAD_DIM = 64
LEAD_QUERIES = 64   # queries per row that attn_prefill_lead recomputes exactly (K4c)


def _p(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need(t: torch.Tensor | None, name: str, dtype: torch.dtype, numel: int | None = None,
          optional: bool = False) -> None:
    if t is None:
        if optional:
            return
        raise ValueError(f"{name} is required")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (got {t.device})")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if numel is not None and t.numel() < numel:
        raise ValueError(f"{name} has {t.numel()} elements, needs {numel}")


LAYOUT_ROWS, LAYOUT_TILES = 0, 1      # MDL_LAYOUT_* of include/mdlarc_hip.h


def _layout(tiled: bool) -> int:
    return LAYOUT_TILES if tiled else LAYOUT_ROWS


def tile_rows(rows: int) -> int:
    """Rows a buffer in the MFMA tile layout holds for ``rows`` rows (whole 16-row blocks)."""
    return (rows + 15) // 16 * 16


def split_numel(rows: int, k: int, tiled: bool) -> int:
    """Elements of a split activation of k channels ([rows, 2k] bf16) in either layout."""
    return (tile_rows(rows) if tiled else rows) * 2 * k


def cache_dtype_code(t: torch.Tensor) -> int:
    """MDL_DTYPE_* of a cache (or q) tensor: bf16 (bf16 form) or fp32 (fp32 form)."""
    if t.dtype == F32:
        return 0
    if t.dtype == BF16:
        return 1
    raise ValueError(f"the KV cache must be bfloat16 or float32 (got {t.dtype})")


def table_dtype_code(t: torch.Tensor) -> int:
    if t.dtype == F32:
        return 0
    if t.dtype == BF16:
        return 1
    raise ValueError(f"embedding tables must be float32 or bfloat16 (got {t.dtype})")


def embed_rmsnorm(ids: torch.Tensor, example_ids: torch.Tensor | None, tok_table: torch.Tensor,
                  ex_table: torch.Tensor | None, row_len: int, gamma: torch.Tensor, eps: float,
                  x_out: torch.Tensor, xs_out: torch.Tensor | None,
                  rstd_out: torch.Tensor | None, tiled: bool = False) -> None:
    """x = tok[ids] + ex[example_ids], rstd, xs = split(x * gamma) as [rows, 2d] bf16; with
    ``tiled`` x in the fp32 and xs in the bf16 MFMA tile layout (the K5 decode entries).
    xs_out and rstd_out may be None."""
    rows = ids.numel()
    vocab, d = tok_table.shape
    _need(ids, "ids", I64)
    _need(example_ids, "example_ids", I64, optional=True)
    _need(tok_table, "tok_table", tok_table.dtype)
    if example_ids is not None:
        _need(ex_table, "ex_table", tok_table.dtype)
        if ex_table.shape[1] != d:
            raise ValueError("example table width differs from token table width")
        if example_ids.numel() * row_len < rows:
            raise ValueError("example_ids shorter than the number of batch rows")
    _need(gamma, "gamma", F32, d)
    _need(x_out, "x_out", F32, (tile_rows(rows) if tiled else rows) * d)
    _need(xs_out, "xs_out", BF16, split_numel(rows, d, tiled), optional=True)
    _need(rstd_out, "rstd_out", F32, rows, optional=True)
    n_ex = ex_table.shape[0] if ex_table is not None else 0
    _lib.check(_lib.lib().mdl_embed_rmsnorm(
        _p(ids), _p(example_ids), _p(tok_table), _p(ex_table), table_dtype_code(tok_table),
        vocab, n_ex, rows, row_len, d, _p(gamma), eps, _p(x_out), _p(xs_out), _p(rstd_out),
        _layout(tiled), _stream()), "mdl_embed_rmsnorm")


def decode_embed(token: torch.Tensor, example_ids: torch.Tensor | None, tok_table: torch.Tensor,
                 ex_table: torch.Tensor | None, gamma: torch.Tensor, eps: float,
                 gx: torch.Tensor, gy: torch.Tensor, in_out: torch.Tensor, pos_out: torch.Tensor,
                 counters: torch.Tensor | None, x_out: torch.Tensor,
                 xs_out: torch.Tensor | None, rstd_out: torch.Tensor | None, max_x: int = 30,
                 max_y: int = 29, tiled: bool = False) -> None:
    """Grid position of each row's emitted token (state advanced), then K1 on that token
    (``tiled`` and the optional outputs as for embed_rmsnorm)."""
    batch = token.numel()
    vocab, d = tok_table.shape
    _need(token, "token", I64)
    _need(example_ids, "example_ids", I64, batch, optional=True)
    _need(tok_table, "tok_table", tok_table.dtype)
    if example_ids is not None:
        _need(ex_table, "ex_table", tok_table.dtype)
        if ex_table.shape[1] != d:
            raise ValueError("example table width differs from token table width")
    for name, t, dt in (("gx", gx, I32), ("gy", gy, I32), ("in_out", in_out, U8)):
        _need(t, name, dt, batch)
    _need(pos_out, "pos_out", I64, batch * 3)
    _need(counters, "counters", I32, 2, optional=True)
    _need(gamma, "gamma", F32, d)
    _need(x_out, "x_out", F32, (tile_rows(batch) if tiled else batch) * d)
    _need(xs_out, "xs_out", BF16, split_numel(batch, d, tiled), optional=True)
    _need(rstd_out, "rstd_out", F32, batch, optional=True)
    n_ex = ex_table.shape[0] if ex_table is not None else 0
    _lib.check(_lib.lib().mdl_decode_embed(
        _p(token), _p(example_ids), _p(tok_table), _p(ex_table), table_dtype_code(tok_table),
        vocab, n_ex, batch, d, _p(gamma), eps, _p(gx), _p(gy), _p(in_out), max_x, max_y,
        _p(pos_out), _p(counters), _p(x_out), _p(xs_out), _p(rstd_out), _layout(tiled),
        _stream()), "mdl_decode_embed")


def add_rmsnorm(x: torch.Tensor, delta: torch.Tensor | None, bias: torch.Tensor | None,
                gamma: torch.Tensor, eps: float, xs_out: torch.Tensor | None,
                rstd_out: torch.Tensor, tiled: bool = False) -> None:
    """x += delta (+ bias) in place (fp32), rstd, xs = split(x * gamma) as [rows, 2d] bf16
    (row-major, or in MFMA tiles when ``tiled``)."""
    rows, d = x.shape
    _need(x, "x", F32)
    _need(delta, "delta", F32, rows * d, optional=True)
    _need(bias, "bias", F32, d, optional=True)
    _need(gamma, "gamma", F32, d)
    _need(xs_out, "xs_out", BF16, split_numel(rows, d, tiled), optional=True)
    _need(rstd_out, "rstd_out", F32, rows)
    _lib.check(_lib.lib().mdl_add_rmsnorm(
        _p(x), _p(delta), _p(bias), rows, d, _p(gamma), eps, _p(xs_out), _p(rstd_out),
        _layout(tiled), _stream()), "mdl_add_rmsnorm")


def qkv_rope_cache(qkv: torch.Tensor, rstd: torch.Tensor | None, pos: torch.Tensor,
                   rope_tab: torch.Tensor, rope_geom: tuple[int, int, int, int, int, int],
                   batch: int, seq: int, n_heads: int, q_scale: float, q_out: torch.Tensor,
                   k_cache: torch.Tensor, v_cache: torch.Tensor, slot0: int = 0,
                   slot_dev: torch.Tensor | None = None) -> None:
    """rope_geom = (max_x, max_y, max_z, px, py, pz); k/v_cache are one layer's
    [batch, n_heads, slots, 64] (contiguous views of the static cache), bf16 or fp32 (the fp32
    form); q_out has the cache's dtype."""
    rows, d = batch * seq, n_heads * HEAD_DIM
    _need(qkv, "qkv", F32, rows * 3 * d)
    if qkv.dim() != 2 or qkv.shape[1] != 3 * d:
        raise ValueError(f"qkv must be [rows, {3 * d}]")
    _need(rstd, "rstd", F32, rows, optional=True)
    _need(pos, "pos", I64, rows * 3)
    _need(rope_tab, "rope_tab", F32)
    dt = cache_dtype_code(k_cache)
    _need(q_out, "q_out", k_cache.dtype, rows * d)
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, k_cache.dtype)
        if c.dim() != 4 or c.shape[0] != batch or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [batch, n_heads, slots, 64]")
    _need(slot_dev, "slot_dev", I32, 1, optional=True)
    slots = k_cache.shape[2]
    mx, my, mz, px, py, pz = rope_geom
    _lib.check(_lib.lib().mdl_qkv_rope_cache(
        _p(qkv), qkv.shape[1], _p(rstd), _p(pos), _p(rope_tab), batch, seq, n_heads, HEAD_DIM,
        mx, my, mz, px, py, pz, q_scale, _p(q_out), _p(k_cache), _p(v_cache), dt, slots, slot0,
        _p(slot_dev), _stream()), "mdl_qkv_rope_cache")


def qkv_rope_cache_packed(qkv: torch.Tensor, rstd: torch.Tensor | None, pos: torch.Tensor,
                          rope_tab: torch.Tensor,
                          rope_geom: tuple[int, int, int, int, int, int],
                          token_row: torch.Tensor, token_slot: torch.Tensor, n_heads: int,
                          q_scale: float, q_out: torch.Tensor, k_cache: torch.Tensor,
                          v_cache: torch.Tensor) -> None:
    """``qkv_rope_cache`` over a packed token list: token m goes to batch row token_row[m],
    cache slot token_slot[m] (no cache write when negative); bf16 or fp32 cache and q_out."""
    rows, d = token_row.numel(), n_heads * HEAD_DIM
    _need(qkv, "qkv", F32, rows * 3 * d)
    if qkv.dim() != 2 or qkv.shape[1] != 3 * d:
        raise ValueError(f"qkv must be [rows, {3 * d}]")
    _need(rstd, "rstd", F32, rows, optional=True)
    _need(pos, "pos", I64, rows * 3)
    _need(rope_tab, "rope_tab", F32)
    dt = cache_dtype_code(k_cache)
    _need(q_out, "q_out", k_cache.dtype, rows * d)
    _need(token_row, "token_row", I32, rows)
    _need(token_slot, "token_slot", I32, rows)
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, k_cache.dtype)
        if c.dim() != 4 or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [batch, n_heads, slots, 64]")
    batch, slots = k_cache.shape[0], k_cache.shape[2]
    mx, my, mz, px, py, pz = rope_geom
    _lib.check(_lib.lib().mdl_qkv_rope_cache_packed(
        _p(qkv), qkv.shape[1], _p(rstd), _p(pos), _p(rope_tab), rows, _p(token_row),
        _p(token_slot), batch, n_heads, HEAD_DIM, mx, my, mz, px, py, pz, q_scale, _p(q_out),
        _p(k_cache), _p(v_cache), dt, slots, _stream()), "mdl_qkv_rope_cache_packed")


def swiglu(gate_up: torch.Tensor, rstd: torch.Tensor | None, bias_gate: torch.Tensor | None,
           bias_up: torch.Tensor | None, h_out: torch.Tensor, tiled: bool = False) -> None:
    """h = silu(rstd*g + b_g) * (rstd*u + b_u) from fp32 gate|up, written as split [rows, 2F]
    (row-major, or in MFMA tiles when ``tiled``)."""
    rows, two_f = gate_up.shape
    f = two_f // 2
    _need(gate_up, "gate_up", F32)
    _need(rstd, "rstd", F32, rows, optional=True)
    _need(bias_gate, "bias_gate", F32, f, optional=True)
    _need(bias_up, "bias_up", F32, f, optional=True)
    _need(h_out, "h_out", BF16, split_numel(rows, f, tiled))
    _lib.check(_lib.lib().mdl_swiglu(
        _p(gate_up), two_f, _p(rstd), _p(bias_gate), _p(bias_up), rows, f, _p(h_out),
        _layout(tiled), _stream()), "mdl_swiglu")


# --- config-1 format (bf16 activations in and out) ----------------------------------------------

def embed_rmsnorm_bf16(ids: torch.Tensor, example_ids: torch.Tensor | None,
                       tok_table: torch.Tensor, ex_table: torch.Tensor | None, row_len: int,
                       gamma: torch.Tensor, eps: float, x_out: torch.Tensor,
                       xn_out: torch.Tensor) -> None:
    """x = bf16(tok[ids] + ex[example_ids]), xn = bf16(x * rstd * gamma), both [rows, d] bf16
    (bf16 tables)."""
    rows = ids.numel()
    vocab, d = tok_table.shape
    _need(ids, "ids", I64)
    _need(example_ids, "example_ids", I64, optional=True)
    _need(tok_table, "tok_table", BF16)
    if example_ids is not None:
        _need(ex_table, "ex_table", BF16)
        if ex_table.shape[1] != d:
            raise ValueError("example table width differs from token table width")
        if example_ids.numel() * row_len < rows:
            raise ValueError("example_ids shorter than the number of batch rows")
    _need(gamma, "gamma", F32, d)
    _need(x_out, "x_out", BF16, rows * d)
    _need(xn_out, "xn_out", BF16, rows * d)
    n_ex = ex_table.shape[0] if ex_table is not None else 0
    _lib.check(_lib.lib().mdl_embed_rmsnorm_bf16(
        _p(ids), _p(example_ids), _p(tok_table), _p(ex_table), vocab, n_ex, rows, row_len, d,
        _p(gamma), eps, _p(x_out), _p(xn_out), _stream()), "mdl_embed_rmsnorm_bf16")


def qkv_rope_cache_bf16(qkv: torch.Tensor, rstd: torch.Tensor | None, pos: torch.Tensor,
                        rope_tab: torch.Tensor, rope_geom: tuple[int, int, int, int, int, int],
                        batch: int, seq: int, n_heads: int, q_scale: float, q_out: torch.Tensor,
                        k_cache: torch.Tensor, v_cache: torch.Tensor, slot0: int = 0) -> None:
    """qkv_rope_cache on a bf16 qkv row [rows, 3d]."""
    rows, d = batch * seq, n_heads * HEAD_DIM
    _need(qkv, "qkv", BF16, rows * 3 * d)
    if qkv.dim() != 2 or qkv.shape[1] != 3 * d:
        raise ValueError(f"qkv must be [rows, {3 * d}]")
    _need(rstd, "rstd", F32, rows, optional=True)
    _need(pos, "pos", I64, rows * 3)
    _need(rope_tab, "rope_tab", F32)
    _need(q_out, "q_out", BF16, rows * d)
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, BF16)
        if c.dim() != 4 or c.shape[0] != batch or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [batch, n_heads, slots, 64]")
    mx, my, mz, px, py, pz = rope_geom
    _lib.check(_lib.lib().mdl_qkv_rope_cache_bf16(
        _p(qkv), qkv.shape[1], _p(rstd), _p(pos), _p(rope_tab), batch, seq, n_heads, HEAD_DIM,
        mx, my, mz, px, py, pz, q_scale, _p(q_out), _p(k_cache), _p(v_cache), k_cache.shape[2],
        slot0, _stream()), "mdl_qkv_rope_cache_bf16")


def swiglu_bf16(gate_up: torch.Tensor, rstd: torch.Tensor | None,
                bias_gate: torch.Tensor | None, bias_up: torch.Tensor | None,
                h_out: torch.Tensor) -> None:
    """h = bf16(silu(rstd*g + b_g) * (rstd*u + b_u)) from bf16 gate|up [rows, 2F] into
    [rows, F] bf16."""
    rows, two_f = gate_up.shape
    f = two_f // 2
    _need(gate_up, "gate_up", BF16)
    _need(rstd, "rstd", F32, rows, optional=True)
    _need(bias_gate, "bias_gate", F32, f, optional=True)
    _need(bias_up, "bias_up", F32, f, optional=True)
    _need(h_out, "h_out", BF16, rows * f)
    _lib.check(_lib.lib().mdl_swiglu_bf16(
        _p(gate_up), two_f, _p(rstd), _p(bias_gate), _p(bias_up), rows, f, _p(h_out),
        _stream()), "mdl_swiglu_bf16")


def gemm_split(a: torch.Tensor, w: torch.Tensor, out: torch.Tensor, k: int,
               a_tiled: bool = False, w_tiled: bool = False, tile: int = 0) -> None:
    """out[m, n] (fp32) = (a_hi + a_lo) @ w[:, :k]^T on the decode GEMM kernel (K5); m, n from
    ``out``.  A row-major ``a`` is [m, >= 2k] (hi | lo), a row-major ``w`` [n, >= k] -- the
    [W | W] operand of gemm_f32 serves, its left half is read.  Tiled operands (MFMA tile
    layout) hold tile_rows(m) * 2k and tile_rows(n) * k elements."""
    _need(a, "a", BF16)
    _need(w, "w", BF16)
    _need(out, "out", F32)
    if out.dim() != 2:
        raise ValueError("out must be [m, n]")
    m, n = out.shape
    lda = ldw = 0
    if a_tiled:
        _need(a, "a", BF16, tile_rows(m) * 2 * k)
    else:
        if a.dim() != 2 or a.shape[0] != m or a.shape[1] < 2 * k:
            raise ValueError(f"a must be [{m}, >= {2 * k}] (got {tuple(a.shape)})")
        lda = a.shape[1]
    if w_tiled:
        _need(w, "w", BF16, tile_rows(n) * k)
    else:
        if w.dim() != 2 or w.shape[0] != n or w.shape[1] < k:
            raise ValueError(f"w must be [{n}, >= {k}] (got {tuple(w.shape)})")
        ldw = w.shape[1]
    _lib.check(_lib.lib().mdl_gemm_split(
        _p(a), lda, _layout(a_tiled), _p(w), ldw, _layout(w_tiled), _p(out), n, m, n, k, tile,
        _stream()), "mdl_gemm_split")


def gemm_split_swiglu(a: torch.Tensor, w_gu: torch.Tensor, rstd: torch.Tensor | None,
                      bias_gate: torch.Tensor | None, bias_up: torch.Tensor | None,
                      h_out: torch.Tensor, m: int, d_ff: int, k: int, tile: int = 0) -> None:
    """h = silu(rstd*g + b_g) * (rstd*u + b_u) straight from the gate / up GEMM (K5 with the
    SwiGLU epilogue): ``a`` tiled split [m, 2k], ``w_gu`` the tiled interleave_gate_up weight,
    ``h_out`` tiled split [m, 2 d_ff]."""
    _need(a, "a", BF16, tile_rows(m) * 2 * k)
    _need(w_gu, "w_gu", BF16, 2 * d_ff * k)
    _need(rstd, "rstd", F32, m, optional=True)
    _need(bias_gate, "bias_gate", F32, d_ff, optional=True)
    _need(bias_up, "bias_up", F32, d_ff, optional=True)
    _need(h_out, "h_out", BF16, split_numel(m, d_ff, True))
    _lib.check(_lib.lib().mdl_gemm_split_swiglu(
        _p(a), _p(w_gu), _p(rstd), _p(bias_gate), _p(bias_up), _p(h_out), m, d_ff, k, tile,
        _stream()), "mdl_gemm_split_swiglu")


def interleave_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """[W_gate; W_up] with their 16-row blocks interleaved (the weight order of
    gemm_split_swiglu): row block 2b = W_gate rows 16b.., row block 2b+1 = W_up rows 16b.."""
    f, k = w_gate.shape
    if tuple(w_up.shape) != (f, k) or f % 16:
        raise ValueError("gate and up weights must be [d_ff, k] with d_ff a multiple of 16")
    return torch.stack([w_gate.reshape(f // 16, 16, k), w_up.reshape(f // 16, 16, k)],
                       1).reshape(2 * f, k).contiguous()


def gemm_norm(x: torch.Tensor, gamma: torch.Tensor, eps: float, w: torch.Tensor,
              out: torch.Tensor, rstd_out: torch.Tensor | None, k: int, tile: int = 0,
              w_lo: torch.Tensor | None = None) -> None:
    """out[m, n] = split(x * gamma) @ W^T with the RMSNorm in K5's prologue; rstd of each row
    into rstd_out (may be None).  x: fp32 tile layout [tile_rows(m), k]; w tiled [n, k].
    w_lo (tiled like w, may be None): the low bf16 part of an fp32 weight (the fp32 form)."""
    _need(out, "out", F32)
    m, n = out.shape
    _need(x, "x", F32, tile_rows(m) * k)
    _need(gamma, "gamma", F32, k)
    _need(w, "w", BF16, tile_rows(n) * k)
    _need(w_lo, "w_lo", BF16, tile_rows(n) * k, optional=True)
    _need(rstd_out, "rstd_out", F32, m, optional=True)
    _lib.check(_lib.lib().mdl_gemm_norm(_p(x), _p(gamma), eps, _p(w), _p(w_lo), _p(out), n,
                                        _p(rstd_out), m, n, k, tile, _stream()),
               "mdl_gemm_norm")


def gemm_norm_qkv(x: torch.Tensor, gamma: torch.Tensor, eps: float, w: torch.Tensor, m: int,
                  n_heads: int, rstd_out: torch.Tensor | None, pos: torch.Tensor,
                  rope_tab: torch.Tensor, rope_geom: tuple[int, int, int, int, int, int],
                  q_scale: float, q_out: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot0: int = 0, slot_dev: torch.Tensor | None = None,
                  tile: int = 0) -> None:
    """ln1 + qkv_proj + K2 of the decode token of each row in one K5 launch: q (bf16 [m, d]),
    K / V into slot slot_dev[0] (or slot0) of each cache row; x the fp32 tile-layout residual
    stream, w the tiled qkv weight."""
    d = n_heads * HEAD_DIM
    _need(x, "x", F32, tile_rows(m) * d)
    _need(gamma, "gamma", F32, d)
    _need(w, "w", BF16, tile_rows(3 * d) * d)
    _need(rstd_out, "rstd_out", F32, m, optional=True)
    _need(pos, "pos", I64, m * 3)
    _need(rope_tab, "rope_tab", F32)
    _need(q_out, "q_out", BF16, m * d)
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, BF16)
        if c.dim() != 4 or c.shape[0] != m or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [m, n_heads, slots, 64]")
    _need(slot_dev, "slot_dev", I32, 1, optional=True)
    mx, my, mz, px, py, pz = rope_geom
    _lib.check(_lib.lib().mdl_gemm_norm_qkv(
        _p(x), _p(gamma), eps, _p(w), m, n_heads, _p(rstd_out), _p(pos), _p(rope_tab), mx, my,
        mz, px, py, pz, q_scale, _p(q_out), _p(k_cache), _p(v_cache), k_cache.shape[2], slot0,
        _p(slot_dev), tile, _stream()), "mdl_gemm_norm_qkv")


def gemm_norm_swiglu(x: torch.Tensor, gamma: torch.Tensor, eps: float, w_gu: torch.Tensor,
                     bias_gate: torch.Tensor | None, bias_up: torch.Tensor | None,
                     h_out: torch.Tensor, m: int, d_ff: int, k: int, tile: int = 0,
                     w_gu_lo: torch.Tensor | None = None) -> None:
    """The gate / up projection of split(x * gamma) (RMSNorm in the prologue) with the SwiGLU
    epilogue: h (tiled split [m, 2 d_ff]).  x: fp32 tile layout; w_gu: tiled
    interleave_gate_up weight; w_gu_lo its low part for an fp32 weight (may be None)."""
    _need(x, "x", F32, tile_rows(m) * k)
    _need(gamma, "gamma", F32, k)
    _need(w_gu, "w_gu", BF16, 2 * d_ff * k)
    _need(w_gu_lo, "w_gu_lo", BF16, 2 * d_ff * k, optional=True)
    _need(bias_gate, "bias_gate", F32, d_ff, optional=True)
    _need(bias_up, "bias_up", F32, d_ff, optional=True)
    _need(h_out, "h_out", BF16, split_numel(m, d_ff, True))
    _lib.check(_lib.lib().mdl_gemm_norm_swiglu(
        _p(x), _p(gamma), eps, _p(w_gu), _p(w_gu_lo), _p(bias_gate), _p(bias_up), _p(h_out), m,
        d_ff, k, tile, _stream()), "mdl_gemm_norm_swiglu")


def gemm_split_residual(a: torch.Tensor, w: torch.Tensor, x: torch.Tensor,
                        bias: torch.Tensor | None, m: int, n: int, k: int,
                        tile: int = 0, w_lo: torch.Tensor | None = None) -> None:
    """x += (a_hi + a_lo) @ W^T (+ bias) in place; a tiled split [m, 2k], w tiled [n, k], x the
    fp32 tile-layout residual stream [tile_rows(m), n]; w_lo the low part of an fp32 w."""
    _need(a, "a", BF16, tile_rows(m) * 2 * k)
    _need(w, "w", BF16, tile_rows(n) * k)
    _need(w_lo, "w_lo", BF16, tile_rows(n) * k, optional=True)
    _need(x, "x", F32, tile_rows(m) * n)
    _need(bias, "bias", F32, n, optional=True)
    _lib.check(_lib.lib().mdl_gemm_split_residual(_p(a), _p(w), _p(w_lo), _p(x), _p(bias), m, n,
                                                  k, tile, _stream()),
               "mdl_gemm_split_residual")


PREFILL_NORM_MAX_K = 2048   # K6 norm forms: gamma is staged in LDS (kMaxNormK)


def _split_a(a: torch.Tensor, m: int, k: int, tiled: bool, parts: int = 2) -> tuple[int, int]:
    """(lda, layout) of an activation [m, parts k] (split hi | lo, or hi alone) in either
    layout."""
    if parts not in (1, 2):
        raise ValueError("a_parts must be 1 (hi) or 2 (hi and lo)")
    if tiled:
        _need(a, "a", BF16, tile_rows(m) * parts * k)
        return parts * k, LAYOUT_TILES
    _need(a, "a", BF16)
    if a.dim() != 2 or a.shape[0] < m or a.shape[1] < parts * k:
        raise ValueError(f"a must be a row-major activation [>= {m}, >= {parts * k}]")
    return a.shape[1], LAYOUT_ROWS


def prefill_gemm_split(a: torch.Tensor, w: torch.Tensor, out: torch.Tensor, k: int,
                       a_tiled: bool = False, a_parts: int = 2) -> None:
    """out[m, n] = (a_hi + a_lo) @ W^T on K6 (prompt-sized rows); w tiled [n, k].  a_parts 1:
    ``a`` holds hi alone ([m, k]) and the product is a_hi @ W^T."""
    _need(out, "out", F32)
    m, n = out.shape
    lda, lay = _split_a(a, m, k, a_tiled, a_parts)
    _need(w, "w", BF16, tile_rows(n) * k)
    _lib.check(_lib.lib().mdl_prefill_gemm_split(_p(a), lda, lay, a_parts, _p(w), _p(out),
                                                 out.stride(0), m, n, k, _stream()),
               "mdl_prefill_gemm_split")


def prefill_gemm_norm(x: torch.Tensor, gamma: torch.Tensor, eps: float, w: torch.Tensor,
                      out: torch.Tensor, rstd_out: torch.Tensor | None, k: int) -> None:
    """out[m, n] = split(x * gamma) @ W^T (RMSNorm in K6's prologue, rstd deferred) and rstd of
    each row; x the fp32 tile-layout residual stream [tile_rows(m), k], w tiled [n, k]."""
    _need(out, "out", F32)
    m, n = out.shape
    _need(x, "x", F32, tile_rows(m) * k)
    _need(gamma, "gamma", F32, k)
    _need(w, "w", BF16, tile_rows(n) * k)
    _need(rstd_out, "rstd_out", F32, m, optional=True)
    _lib.check(_lib.lib().mdl_prefill_gemm_norm(_p(x), _p(gamma), eps, _p(w), _p(out),
                                                out.stride(0), _p(rstd_out), m, n, k,
                                                _stream()), "mdl_prefill_gemm_norm")


def prefill_gemm_norm_swiglu(x: torch.Tensor, gamma: torch.Tensor, eps: float,
                             w_gu: torch.Tensor, bias_gate: torch.Tensor | None,
                             bias_up: torch.Tensor | None, h_out: torch.Tensor, m: int,
                             d_ff: int, k: int, a_parts: int = 2, h_parts: int = 2) -> None:
    """h (tiled [m, h_parts d_ff]: hi, then lo when h_parts is 2) = SwiGLU of the gate / up
    projection of split(x * gamma) (a_parts 1: of bf16(x * gamma)); x the fp32 tile-layout
    residual stream, w_gu the tiled interleave_gate_up weight."""
    if a_parts not in (1, 2) or h_parts not in (1, 2):
        raise ValueError("a_parts and h_parts must be 1 (hi) or 2 (hi and lo)")
    _need(x, "x", F32, tile_rows(m) * k)
    _need(gamma, "gamma", F32, k)
    _need(w_gu, "w_gu", BF16, 2 * d_ff * k)
    _need(bias_gate, "bias_gate", F32, d_ff, optional=True)
    _need(bias_up, "bias_up", F32, d_ff, optional=True)
    _need(h_out, "h_out", BF16, tile_rows(m) * h_parts * d_ff)
    _lib.check(_lib.lib().mdl_prefill_gemm_norm_swiglu(
        _p(x), _p(gamma), eps, a_parts, _p(w_gu), _p(bias_gate), _p(bias_up), _p(h_out),
        h_parts, m, d_ff, k, _stream()), "mdl_prefill_gemm_norm_swiglu")


def prefill_gemm_split_residual(a: torch.Tensor, w: torch.Tensor, x: torch.Tensor,
                                bias: torch.Tensor | None, m: int, n: int, k: int,
                                a_tiled: bool = False, a_parts: int = 2) -> None:
    """x += (a_hi + a_lo) @ W^T (+ bias) in place; x the fp32 tile-layout residual stream
    [tile_rows(m), n], w tiled [n, k], a split [m, 2k] row-major or tiled (a_parts 1: hi alone,
    [m, k], and x += a_hi @ W^T)."""
    lda, lay = _split_a(a, m, k, a_tiled, a_parts)
    _need(x, "x", F32, tile_rows(m) * n)
    _need(w, "w", BF16, tile_rows(n) * k)
    _need(bias, "bias", F32, n, optional=True)
    _lib.check(_lib.lib().mdl_prefill_gemm_split_residual(_p(a), lda, lay, a_parts, _p(w),
                                                          _p(x), _p(bias), m, n, k, _stream()),
               "mdl_prefill_gemm_split_residual")


def prefill_gemm_norm_qkv(x: torch.Tensor, gamma: torch.Tensor, eps: float, w: torch.Tensor,
                          rows: int, n_heads: int, rstd_out: torch.Tensor | None,
                          qkv_lead: torch.Tensor | None, lead: int,
                          kv_start: torch.Tensor | None, pos: torch.Tensor,
                          rope_tab: torch.Tensor,
                          rope_geom: tuple[int, int, int, int, int, int], q_scale: float,
                          q_out: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                          token_row: torch.Tensor | None = None,
                          token_slot: torch.Tensor | None = None, seq: int = 0) -> None:
    """ln1 + qkv_proj + K2 in one K6 launch: q (bf16 [rows, d]) and K / V into their cache slots
    as qkv_rope_cache(_packed) writes them from the same projection, rstd of each row, and the
    fp32 projection rows of each batch row's first ``lead`` tokens (from kv_start) into qkv_lead
    (may be None).  Rows are a packed token list (token_row / token_slot) or [batch, seq]."""
    d = n_heads * HEAD_DIM
    _need(x, "x", F32, tile_rows(rows) * d)
    _need(gamma, "gamma", F32, d)
    _need(w, "w", BF16, tile_rows(3 * d) * d)
    _need(rstd_out, "rstd_out", F32, rows, optional=True)
    _need(qkv_lead, "qkv_lead", F32, rows * 3 * d, optional=True)
    if qkv_lead is not None and (qkv_lead.dim() != 2 or qkv_lead.shape[1] != 3 * d):
        raise ValueError(f"qkv_lead must be [rows, {3 * d}]")
    _need(pos, "pos", I64, rows * 3)
    _need(rope_tab, "rope_tab", F32)
    _need(q_out, "q_out", BF16, rows * d)
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, BF16)
        if c.dim() != 4 or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [batch, n_heads, slots, 64]")
    batch, slots = k_cache.shape[0], k_cache.shape[2]
    _need(kv_start, "kv_start", I32, batch, optional=True)
    if (token_row is None) != (token_slot is None):
        raise ValueError("token_row and token_slot go together")
    if token_row is not None:
        _need(token_row, "token_row", I32, rows)
        _need(token_slot, "token_slot", I32, rows)
    elif seq * batch != rows:
        raise ValueError("unpacked rows need rows == batch * seq")
    mx, my, mz, px, py, pz = rope_geom
    _lib.check(_lib.lib().mdl_prefill_gemm_norm_qkv(
        _p(x), _p(gamma), eps, _p(w), rows, n_heads, _p(rstd_out), _p(qkv_lead), 3 * d, lead,
        _p(kv_start), _p(pos), _p(rope_tab), mx, my, mz, px, py, pz, q_scale, _p(q_out),
        _p(k_cache), _p(v_cache), slots, batch, seq, _p(token_row), _p(token_slot), _stream()),
        "mdl_prefill_gemm_norm_qkv")


def tile_f32(x: torch.Tensor) -> torch.Tensor:
    """[rows, cols] fp32 (cols a multiple of 32) in the fp32 tile layout: a new flat tensor of
    tile_rows(rows) * cols floats, padding rows zero (torch ops; for tests and set-up)."""
    rows, cols = x.shape
    if cols % 32:
        raise ValueError("the fp32 tile layout needs a multiple of 32 columns")
    xp = torch.zeros(tile_rows(rows), cols, dtype=x.dtype, device=x.device)
    xp[:rows] = x
    # [row block, r, col block, q, h, e] -> [row block, col block, h, q, r, e]
    return xp.view(-1, 16, cols // 32, 4, 2, 4).permute(0, 2, 4, 3, 1, 5).reshape(-1)


def untile_f32(t: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """The inverse of tile_f32: the [rows, cols] matrix."""
    v = t[:tile_rows(rows) * cols].view(-1, cols // 32, 2, 4, 16, 4)
    return v.permute(0, 4, 1, 3, 2, 5).reshape(-1, cols)[:rows]


def untile_matrix(t: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """The inverse of tile_matrix for a bf16 buffer: the [rows, cols] matrix (torch ops; for
    tests and tools)."""
    v = t.reshape(-1)[:tile_rows(rows) * cols].view(-1, cols // 32, 4, 16, 8)
    return v.permute(0, 3, 1, 2, 4).reshape(-1, cols)[:rows]


def gemm_split_tiles() -> int:
    return _lib.lib().mdl_gemm_split_tiles()


def gemm_split_pick(m: int, n: int, k: int) -> int:
    return _lib.lib().mdl_gemm_split_pick(m, n, k)


def tile_matrix(src: torch.Tensor, cols: int | None = None) -> torch.Tensor:
    """Columns [0, cols) of the 2-D bf16 ``src`` in the MFMA tile layout (a new flat tensor of
    tile_rows(rows) * cols elements; padding rows zero)."""
    _need(src, "src", BF16)
    if src.dim() != 2:
        raise ValueError("src must be 2-D")
    rows = src.shape[0]
    cols = src.shape[1] if cols is None else cols
    dst = torch.empty(tile_rows(rows) * cols, dtype=BF16, device=src.device)
    _lib.check(_lib.lib().mdl_tile_matrix(_p(src), src.shape[1], rows, cols, _p(dst),
                                          _stream()), "mdl_tile_matrix")
    return dst


def attn_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, batch: int,
                 seq: int, n_heads: int, key_mask: torch.Tensor | None,
                 kv_start: torch.Tensor | None, causal: bool, out: torch.Tensor,
                 out_tiled: bool = False, row_holes: torch.Tensor | None = None) -> None:
    """out: split [batch*seq, 2*n_heads*64] bf16 (row-major, or the MFMA tile layout).
    row_holes (uint8 [batch], from grid_init): 0 marks a row whose key mask is exactly
    [kv_start, seq), which the kernel then does not read."""
    n = batch * seq * n_heads * HEAD_DIM
    _need(q, "q", BF16, n)
    _need(out, "out", BF16, split_numel(batch * seq, n_heads * HEAD_DIM, out_tiled))
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, BF16)
        if c.dim() != 4 or c.shape[0] != batch or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [batch, n_heads, slots, 64]")
    _need(key_mask, "key_mask", U8, batch * seq, optional=True)
    _need(row_holes, "row_holes", U8, batch, optional=True)
    _need(kv_start, "kv_start", I32, batch, optional=True)
    _lib.check(_lib.lib().mdl_attn_prefill(
        _p(q), _p(k_cache), _p(v_cache), batch, seq, n_heads, HEAD_DIM, k_cache.shape[2],
        _p(key_mask), _p(row_holes), _p(kv_start), 1 if causal else 0, _p(out),
        _layout(out_tiled), _stream()), "mdl_attn_prefill")


def attn_prefill_packed(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        batch: int, seq: int, n_heads: int, key_mask: torch.Tensor | None,
                        kv_start: torch.Tensor, q_offset: torch.Tensor, n_rows: int,
                        causal: bool, out: torch.Tensor, out_tiled: bool = False,
                        row_holes: torch.Tensor | None = None) -> None:
    """Packed query rows: query i >= kv_start[b] of row b is row q_offset[b] + i - kv_start[b]
    of q ([n_rows, n_heads*64]) and out (split [n_rows, 2*n_heads*64], row-major or tiled).
    The caller guarantees q_offset[b] + seq - kv_start[b] <= n_rows for every row.  row_holes
    as in attn_prefill."""
    n = n_rows * n_heads * HEAD_DIM
    _need(q, "q", BF16, n)
    _need(out, "out", BF16, split_numel(n_rows, n_heads * HEAD_DIM, out_tiled))
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, BF16)
        if c.dim() != 4 or c.shape[0] != batch or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [batch, n_heads, slots, 64]")
    _need(key_mask, "key_mask", U8, batch * seq, optional=True)
    _need(row_holes, "row_holes", U8, batch, optional=True)
    _need(kv_start, "kv_start", I32, batch)
    _need(q_offset, "q_offset", I32, batch)
    _lib.check(_lib.lib().mdl_attn_prefill_packed(
        _p(q), _p(k_cache), _p(v_cache), batch, seq, n_heads, HEAD_DIM, k_cache.shape[2],
        _p(key_mask), _p(row_holes), _p(kv_start), _p(q_offset), 1 if causal else 0, _p(out),
        _layout(out_tiled), _stream()), "mdl_attn_prefill_packed")


def _f32_cache(k_cache: torch.Tensor, v_cache: torch.Tensor, batch: int, n_heads: int) -> None:
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, F32)
        if c.dim() != 4 or c.shape[0] != batch or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [batch, n_heads, slots, 64]")


def attn_prefill_f32(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, batch: int,
                     seq: int, n_heads: int, key_mask: torch.Tensor | None,
                     kv_start: torch.Tensor | None, q_offset: torch.Tensor | None, n_rows: int,
                     causal: bool, out: torch.Tensor, out_tiled: bool = False) -> None:
    """K4f, the fp32 form's attention over keys [0, seq) of an fp32 cache: q fp32
    [n_rows, n_heads*64] (rows b*seq + i, or packed through q_offset / kv_start as in
    attn_prefill_packed), out split [n_rows, 2*n_heads*64] bf16 (row-major or tiled)."""
    _need(q, "q", F32, n_rows * n_heads * HEAD_DIM)
    _need(out, "out", BF16, split_numel(n_rows, n_heads * HEAD_DIM, out_tiled))
    _f32_cache(k_cache, v_cache, batch, n_heads)
    _need(key_mask, "key_mask", U8, batch * seq, optional=True)
    _need(kv_start, "kv_start", I32, batch, optional=q_offset is None)
    _need(q_offset, "q_offset", I32, batch, optional=True)
    if q_offset is None and n_rows < batch * seq:
        raise ValueError("unpacked queries need n_rows >= batch * seq")
    _lib.check(_lib.lib().mdl_attn_prefill_f32(
        _p(q), _p(k_cache), _p(v_cache), batch, seq, n_heads, HEAD_DIM, k_cache.shape[2],
        _p(key_mask), _p(kv_start), _p(q_offset), 1 if causal else 0, _p(out),
        _layout(out_tiled), _stream()), "mdl_attn_prefill_f32")


def attn_decode_f32(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, batch: int,
                    n_heads: int, prompt_mask: torch.Tensor | None, prompt_len: int,
                    kv_start: torch.Tensor | None, seq_pos: int, seq_dev: torch.Tensor | None,
                    workspace: torch.Tensor | None, split_len: int, out: torch.Tensor,
                    tiled: bool = False) -> None:
    """K4f at decode: the query of row b (fp32 q [batch, n_heads*64]) over slots
    [kv_start[b], t] of the fp32 cache, t = seq_dev[0] (or seq_pos), the prompt mask applying
    below prompt_len; out split [batch, 2*n_heads*64] bf16.  The slots go in chunks of
    ``split_len`` (a multiple of 16), one wave each; with more than one chunk their states are
    merged through ``workspace`` (attn_decode_workspace_bytes(batch, n_heads, slots,
    split_len) bytes)."""
    _need(q, "q", F32, batch * n_heads * HEAD_DIM)
    _need(out, "out", BF16, split_numel(batch, n_heads * HEAD_DIM, tiled))
    _f32_cache(k_cache, v_cache, batch, n_heads)
    _need(prompt_mask, "prompt_mask", U8, batch * prompt_len, optional=True)
    _need(kv_start, "kv_start", I32, batch, optional=True)
    _need(seq_dev, "seq_dev", I32, 1, optional=True)
    _need(workspace, "workspace", F32, optional=True)
    ws_bytes = workspace.numel() * 4 if workspace is not None else 0
    _lib.check(_lib.lib().mdl_attn_decode_f32(
        _p(q), _p(k_cache), _p(v_cache), batch, n_heads, HEAD_DIM, k_cache.shape[2],
        _p(prompt_mask), prompt_len, _p(kv_start), seq_pos, _p(seq_dev), _p(workspace),
        ws_bytes, split_len, _p(out), _layout(tiled), _stream()), "mdl_attn_decode_f32")


def attn_prefill_lead(qkv: torch.Tensor, rstd: torch.Tensor, pos: torch.Tensor,
                      rope_tab: torch.Tensor, rope_geom: tuple[int, int, int, int, int, int],
                      q_scale: float, batch: int, seq: int, n_heads: int,
                      key_mask: torch.Tensor | None, kv_start: torch.Tensor | None,
                      q_offset: torch.Tensor | None, n_rows: int, out: torch.Tensor,
                      out_tiled: bool = False) -> None:
    """Exact fp32 causal attention for the first 64 queries at or after kv_start of each row,
    overwriting those rows of ``out`` (after attn_prefill / attn_prefill_packed).  ``qkv`` /
    ``rstd`` / ``pos`` hold the n_rows token rows K2 consumed; rows are [batch, seq] or, with
    q_offset, packed."""
    d = n_heads * HEAD_DIM
    _need(qkv, "qkv", F32, n_rows * 3 * d)
    if qkv.dim() != 2 or qkv.shape[1] != 3 * d:
        raise ValueError(f"qkv must be [rows, {3 * d}]")
    _need(rstd, "rstd", F32, n_rows)
    _need(pos, "pos", I64, n_rows * 3)
    _need(rope_tab, "rope_tab", F32)
    _need(out, "out", BF16, split_numel(n_rows, d, out_tiled))
    _need(key_mask, "key_mask", U8, batch * seq, optional=True)
    _need(kv_start, "kv_start", I32, batch, optional=q_offset is None)
    _need(q_offset, "q_offset", I32, batch, optional=True)
    if q_offset is None and n_rows < batch * seq:
        raise ValueError("unpacked rows need batch * seq rows")
    mx, my, mz, px, py, pz = rope_geom
    _lib.check(_lib.lib().mdl_attn_prefill_lead(
        _p(qkv), qkv.shape[1], _p(rstd), _p(pos), _p(rope_tab), mx, my, mz, px, py, pz, q_scale,
        batch, seq, n_heads, HEAD_DIM, _p(key_mask), _p(kv_start), _p(q_offset), _p(out),
        _layout(out_tiled), _stream()), "mdl_attn_prefill_lead")


def attn_decode_workspace_bytes(batch: int, n_heads: int, slots: int, split_len: int) -> int:
    return int(_lib.lib().mdl_attn_decode_workspace_bytes(batch, n_heads, slots, split_len))


def attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, batch: int,
                n_heads: int, prompt_mask: torch.Tensor | None, prompt_len: int,
                kv_start: torch.Tensor | None, seq_pos: int, seq_dev: torch.Tensor | None,
                workspace: torch.Tensor | None, split_len: int, out: torch.Tensor,
                row_holes: torch.Tensor | None = None,
                row_order: torch.Tensor | None = None, tiled: bool = False) -> None:
    """out: split [batch, 2*n_heads*64] bf16 (row-major, or MFMA tiles when ``tiled``).
    row_holes (uint8 [batch], from grid_init): rows marked 0 skip the prompt-mask reads.
    row_order (int32 [batch]): permutation giving the dispatch order of the rows (longest
    first)."""
    n = batch * n_heads * HEAD_DIM
    _need(q, "q", BF16, n)
    _need(out, "out", BF16, split_numel(batch, n_heads * HEAD_DIM, tiled))
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, BF16)
        if c.dim() != 4 or c.shape[0] != batch or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [batch, n_heads, slots, 64]")
    _need(prompt_mask, "prompt_mask", U8, batch * prompt_len, optional=True)
    _need(row_holes, "row_holes", U8, batch, optional=True)
    _need(kv_start, "kv_start", I32, batch, optional=True)
    _need(row_order, "row_order", I32, batch, optional=True)
    _need(seq_dev, "seq_dev", I32, 1, optional=True)
    _need(workspace, "workspace", F32, optional=True)
    ws_bytes = 0 if workspace is None else workspace.numel() * 4
    _lib.check(_lib.lib().mdl_attn_decode(
        _p(q), _p(k_cache), _p(v_cache), batch, n_heads, HEAD_DIM, k_cache.shape[2],
        _p(prompt_mask), prompt_len, _p(row_holes), _p(kv_start), _p(row_order), seq_pos,
        _p(seq_dev),
        _p(workspace), ws_bytes, split_len, _p(out), _layout(tiled), _stream()),
        "mdl_attn_decode")


def attn_decode_rope(qkv: torch.Tensor, rstd: torch.Tensor, pos: torch.Tensor,
                     rope_tab: torch.Tensor, rope_geom: tuple[int, int, int, int, int, int],
                     q_scale: float, k_cache: torch.Tensor, v_cache: torch.Tensor, batch: int,
                     n_heads: int, prompt_mask: torch.Tensor | None, prompt_len: int,
                     kv_start: torch.Tensor | None, seq_pos: int, seq_dev: torch.Tensor | None,
                     workspace: torch.Tensor | None, split_len: int, out: torch.Tensor,
                     row_holes: torch.Tensor | None = None,
                     row_order: torch.Tensor | None = None, tiled: bool = False) -> None:
    """qkv_rope_cache (one token per row, slot t) + attn_decode in one launch."""
    d = n_heads * HEAD_DIM
    _need(qkv, "qkv", F32, batch * 3 * d)
    if qkv.dim() != 2 or qkv.shape[1] != 3 * d:
        raise ValueError(f"qkv must be [batch, {3 * d}]")
    _need(rstd, "rstd", F32, batch)
    _need(pos, "pos", I64, batch * 3)
    _need(rope_tab, "rope_tab", F32)
    _need(out, "out", BF16, split_numel(batch, d, tiled))
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, BF16)
        if c.dim() != 4 or c.shape[0] != batch or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [batch, n_heads, slots, 64]")
    _need(prompt_mask, "prompt_mask", U8, batch * prompt_len, optional=True)
    _need(row_holes, "row_holes", U8, batch, optional=True)
    _need(kv_start, "kv_start", I32, batch, optional=True)
    _need(row_order, "row_order", I32, batch, optional=True)
    _need(seq_dev, "seq_dev", I32, 1, optional=True)
    _need(workspace, "workspace", F32, optional=True)
    ws_bytes = 0 if workspace is None else workspace.numel() * 4
    mx, my, mz, px, py, pz = rope_geom
    _lib.check(_lib.lib().mdl_attn_decode_rope(
        _p(qkv), qkv.shape[1], _p(rstd), _p(pos), _p(rope_tab), mx, my, mz, px, py, pz, q_scale,
        _p(k_cache), _p(v_cache), batch, n_heads, HEAD_DIM, k_cache.shape[2], _p(prompt_mask),
        prompt_len, _p(row_holes), _p(kv_start), _p(row_order), seq_pos, _p(seq_dev),
        _p(workspace), ws_bytes, split_len, _p(out), _layout(tiled), _stream()),
        "mdl_attn_decode_rope")


DECODE_SCRATCH_BYTES = 4 << 20   # MDL_DECODE_SCRATCH_BYTES


def attn_decode_rope_noalloc(qkv: torch.Tensor, rstd: torch.Tensor, pos: torch.Tensor,
                             rope_tab: torch.Tensor,
                             rope_geom: tuple[int, int, int, int, int, int], q_scale: float,
                             k_cache: torch.Tensor, v_cache: torch.Tensor, batch: int,
                             n_heads: int, prompt_mask: torch.Tensor | None, prompt_len: int,
                             kv_start: torch.Tensor | None, seq_pos: int,
                             seq_dev: torch.Tensor | None, split_len: int, out: torch.Tensor,
                             row_holes: torch.Tensor | None = None,
                             row_order: torch.Tensor | None = None, tiled: bool = False) -> None:
    """attn_decode_rope with its split partials in the library's static per-GPU scratch buffer
    (DECODE_SCRATCH_BYTES) instead of a workspace tensor: allocates nothing.  Calls on one GPU
    share that buffer, so calls that overlap in time on one GPU race."""
    d = n_heads * HEAD_DIM
    _need(qkv, "qkv", F32, batch * 3 * d)
    if qkv.dim() != 2 or qkv.shape[1] != 3 * d:
        raise ValueError(f"qkv must be [batch, {3 * d}]")
    _need(rstd, "rstd", F32, batch)
    _need(pos, "pos", I64, batch * 3)
    _need(rope_tab, "rope_tab", F32)
    _need(out, "out", BF16, split_numel(batch, d, tiled))
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, BF16)
        if c.dim() != 4 or c.shape[0] != batch or c.shape[1] != n_heads or c.shape[3] != 64:
            raise ValueError(f"{name} must be [batch, n_heads, slots, 64]")
    _need(prompt_mask, "prompt_mask", U8, batch * prompt_len, optional=True)
    _need(row_holes, "row_holes", U8, batch, optional=True)
    _need(kv_start, "kv_start", I32, batch, optional=True)
    _need(row_order, "row_order", I32, batch, optional=True)
    _need(seq_dev, "seq_dev", I32, 1, optional=True)
    mx, my, mz, px, py, pz = rope_geom
    _lib.check(_lib.lib().mdl_attn_decode_rope_noalloc(
        _p(qkv), qkv.shape[1], _p(rstd), _p(pos), _p(rope_tab), mx, my, mz, px, py, pz, q_scale,
        _p(k_cache), _p(v_cache), batch, n_heads, HEAD_DIM, k_cache.shape[2], _p(prompt_mask),
        prompt_len, _p(row_holes), _p(kv_start), _p(row_order), seq_pos, _p(seq_dev),
        split_len, _p(out), _layout(tiled), _stream()),
        "mdl_attn_decode_rope_noalloc")


class HeadConstraints:
    """Device form of DecodingConstraints for the head kernels (``mdl_logit_constraints``):
    keeps the tensors it points at alive for as long as the launches (or a captured graph)
    use them.  palette uint8/bool [rows, 10] and target_shape int [rows, 2] may be None; gx / gy
    are the decode state's grid position (int32 [rows]), read at launch time."""

    def __init__(self, disallow_tokens, palette: torch.Tensor | None, palette_penalty: float,
                 target_shape: torch.Tensor | None, gx: torch.Tensor, gy: torch.Tensor,
                 shape_penalty: float):
        rows = gx.numel()
        self.palette = None if palette is None else palette.to(torch.uint8).contiguous()
        self.shape = None if target_shape is None else target_shape.to(torch.int32).contiguous()
        _need(self.palette, "palette", U8, rows * 10, optional=True)
        _need(self.shape, "target_shape", I32, rows * 2, optional=True)
        _need(gx, "gx", I32, rows)
        _need(gy, "gy", I32, rows)
        self.gx, self.gy, self.rows = gx, gy, rows
        mask = 0
        for t in disallow_tokens:
            if not 0 <= int(t) < 32:
                raise ValueError(f"disallowed token {t} outside the head's 32 vocab slots")
            mask |= 1 << int(t)
        addr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        self.struct = _lib.LogitConstraints(mask, addr(self.palette), float(palette_penalty),
                                            addr(self.shape), addr(gx), addr(gy),
                                            float(shape_penalty))

    def ref(self, rows: int):
        if rows != self.rows:
            raise ValueError(f"constraints built for {self.rows} rows, launch has {rows}")
        return ctypes.byref(self.struct)


def lm_head(x: torch.Tensor, row_index: torch.Tensor | None, rows: int, gamma: torch.Tensor,
            eps: float, w_head: torch.Tensor, logits_out: torch.Tensor | None,
            token_out: torch.Tensor | None, constraints: HeadConstraints | None = None,
            x_tiled: bool = False) -> None:
    """x: [rows, d] fp32, row-major or (``x_tiled``) in the fp32 tile layout."""
    d = x.shape[-1]
    vocab = w_head.shape[0]
    _need(x, "x", F32)
    _need(row_index, "row_index", I32, rows, optional=True)
    if row_index is None and x.numel() < (tile_rows(rows) if x_tiled else rows) * d:
        raise ValueError("x has fewer rows than requested")
    _need(gamma, "gamma", F32, d)
    _need(w_head, "w_head", F32, vocab * d)
    _need(logits_out, "logits_out", F32, rows * vocab, optional=True)
    _need(token_out, "token_out", I64, rows, optional=True)
    _lib.check(_lib.lib().mdl_lm_head(
        _p(x), _p(row_index), rows, d, _p(gamma), eps, _p(w_head), vocab, _p(logits_out),
        _p(token_out), None if constraints is None else constraints.ref(rows), _layout(x_tiled),
        _stream()), "mdl_lm_head")


def decode_head(x: torch.Tensor, gamma: torch.Tensor, eps: float, w_head: torch.Tensor,
                logits_out: torch.Tensor | None, token_out: torch.Tensor, out_ids: torch.Tensor,
                col: int, counters: torch.Tensor | None, finish_step: torch.Tensor | None,
                gen_base: int, end_id: int, constraints: HeadConstraints | None = None,
                x_tiled: bool = False) -> None:
    """ln_f + LM head (+ constraints) + argmax into token_out, committed to
    out_ids[:, counters[1] or col].  x: [batch, d] fp32, or (``x_tiled``) the fp32 tile layout
    with tile_rows(batch) rows."""
    batch, d = token_out.numel(), x.shape[-1]
    vocab = w_head.shape[0]
    _need(x, "x", F32, (tile_rows(batch) if x_tiled else batch) * d)
    _need(gamma, "gamma", F32, d)
    _need(w_head, "w_head", F32, vocab * d)
    _need(logits_out, "logits_out", F32, batch * vocab, optional=True)
    _need(token_out, "token_out", I64, batch)
    _need(out_ids, "out_ids", I64)
    if out_ids.dim() != 2 or out_ids.shape[0] != batch:
        raise ValueError("out_ids must be [batch, columns]")
    _need(counters, "counters", I32, 2, optional=True)
    _need(finish_step, "finish_step", I32, batch, optional=True)
    _lib.check(_lib.lib().mdl_decode_head(
        _p(x), batch, d, _p(gamma), eps, _p(w_head), vocab, _p(logits_out), _p(token_out),
        _p(out_ids), out_ids.shape[1], col, _p(counters), _p(finish_step), gen_base, end_id,
        None if constraints is None else constraints.ref(batch), _layout(x_tiled), _stream()),
        "mdl_decode_head")


def grid_init(ids: torch.Tensor, pos: torch.Tensor, mask: torch.Tensor | None, gx: torch.Tensor,
              gy: torch.Tensor, in_out: torch.Tensor, kv_start: torch.Tensor | None,
              last_row: torch.Tensor | None, max_x: int = 30, max_y: int = 29,
              row_holes: torch.Tensor | None = None,
              row_shift: torch.Tensor | None = None) -> None:
    """row_shift (int32 [batch]): extra left padding of each row relative to the batch the
    reference padded it in (its lengths-1 index moves by that much); None = 0."""
    batch, seq = ids.shape
    _need(ids, "ids", I64)
    _need(pos, "pos", I64, batch * seq * 3)
    _need(mask, "mask", U8, batch * seq, optional=True)
    _need(gx, "gx", I32, batch)
    _need(gy, "gy", I32, batch)
    _need(in_out, "in_out", U8, batch)
    _need(kv_start, "kv_start", I32, batch, optional=True)
    _need(last_row, "last_row", I32, batch, optional=True)
    _need(row_holes, "row_holes", U8, batch, optional=True)
    _need(row_shift, "row_shift", I32, batch, optional=True)
    _lib.check(_lib.lib().mdl_grid_init(
        _p(ids), _p(pos), _p(mask), _p(row_shift), batch, seq, max_x, max_y, _p(gx), _p(gy),
        _p(in_out), _p(kv_start), _p(last_row), _p(row_holes), _stream()), "mdl_grid_init")


def grid_step(token: torch.Tensor, gx: torch.Tensor, gy: torch.Tensor, in_out: torch.Tensor,
              pos_out: torch.Tensor, counters: torch.Tensor | None, max_x: int = 30,
              max_y: int = 29) -> None:
    batch = token.numel()
    _need(token, "token", I64)
    _need(gx, "gx", I32, batch)
    _need(gy, "gy", I32, batch)
    _need(in_out, "in_out", U8, batch)
    _need(pos_out, "pos_out", I64, batch * 3)
    _need(counters, "counters", I32, 2, optional=True)
    _lib.check(_lib.lib().mdl_grid_step(
        _p(token), batch, max_x, max_y, _p(gx), _p(gy), _p(in_out), _p(pos_out), _p(counters),
        _stream()), "mdl_grid_step")


def build_prompts(cells: torch.Tensor, grids: torch.Tensor, variants: torch.Tensor,
                  perms: torch.Tensor, lengths: torch.Tensor, ids_out: torch.Tensor,
                  pos_out: torch.Tensor, mask_out: torch.Tensor) -> None:
    """Augmented prompts of one task into the left-padded batch (mdl_build_prompts): cells uint8
    (all grids row-major), grids int32 [n, 3] (offset, h, w), variants int32 [B, 2] (dihedral,
    perm row), perms int32 [P, 10], lengths int32 [B]; ids int64 / pos int64 [B, S, 3] / mask
    uint8 [B, S]."""
    batch, seq = ids_out.shape
    _need(cells, "cells", U8)
    _need(grids, "grids", I32)
    _need(variants, "variants", I32, batch * 2)
    _need(perms, "perms", I32)
    _need(lengths, "lengths", I32, batch)
    _need(ids_out, "ids_out", I64, batch * seq)
    _need(pos_out, "pos_out", I64, batch * seq * 3)
    _need(mask_out, "mask_out", U8, batch * seq)
    if grids.dim() != 2 or grids.shape[1] != 3 or perms.dim() != 2 or perms.shape[1] != 10:
        raise ValueError("grids must be [n, 3] and perms [P, 10]")
    _lib.check(_lib.lib().mdl_build_prompts(
        _p(cells), cells.numel(), _p(grids), grids.shape[0], _p(variants), batch, _p(perms),
        perms.shape[0], _p(lengths), seq, _p(ids_out), _p(pos_out), _p(mask_out), _stream()),
        "mdl_build_prompts")


def decode_commit(token: torch.Tensor, out_ids: torch.Tensor, col: int,
                  counters: torch.Tensor | None, finish_step: torch.Tensor | None,
                  gen_base: int, end_id: int) -> None:
    batch = token.numel()
    _need(token, "token", I64)
    _need(out_ids, "out_ids", I64)
    if out_ids.dim() != 2 or out_ids.shape[0] != batch:
        raise ValueError("out_ids must be [batch, columns]")
    _need(counters, "counters", I32, 2, optional=True)
    _need(finish_step, "finish_step", I32, batch, optional=True)
    _lib.check(_lib.lib().mdl_decode_commit(
        _p(token), batch, _p(out_ids), out_ids.shape[1], col, _p(counters), _p(finish_step),
        gen_base, end_id, _stream()), "mdl_decode_commit")
