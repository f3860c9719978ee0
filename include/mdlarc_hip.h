/*
 * mdlarc_hip.h -- C ABI of libmdlarc_hip.so, the MI355X (gfx950) kernels of the TinyTransformer
 * inference hot path of shyampathak22/mdlARC_scale.
 *
 * The reference has no FFI: its boundary is the PyTorch module / function API of
 * src/transformer.py and src/inference.py.  Each entry point below replaces the reference ops
 * named in its comment (file:line in the reference checkout).  The host side
 * (mdlarc_scale_amd/_lib.py, Python) binds these with ctypes.
 *
 * Conventions
 *   - bf16 tensors are passed as uint16_t* (raw bfloat16 bits), fp32 as float*.
 *   - Every pointer is a DEVICE pointer unless stated otherwise; `stream` is a hipStream_t.
 *   - Nothing allocates, frees or synchronises; all work is ordered on `stream`.
 *   - Return 0 on success, a negative MDL_ERR_* for arguments rejected on the host before any
 *     launch, or a positive hipError_t reported by the launch.
 *   - Head dimension is 64 (all reference model sizes, src/transformer.py:728-745).
 *   - GEMM inputs ("split activations") are written as hi|lo bf16 pairs: a row of K values is 2K
 *     bf16, hi = bf16(v) in columns [0, K), lo = bf16(v - hi) in [K, 2K).  Multiplied with a
 *     weight packed as [W | W] ([N, 2K] bf16) a bf16 GEMM with fp32 accumulation returns
 *     (hi + lo) . w, i.e. the fp32 activation against the bf16 weight.  GEMM outputs are
 *     consumed in fp32.
 *   - MDL_LAYOUT_TILES stores a [rows, C] bf16 matrix (C a multiple of 32; the split
 *     activation has C = 2K) as 16 x 32 blocks of 1 KB, block (r / 16, c / 32) at element
 *     512 * ((r / 16) * (C / 32) + c / 32); inside a block, row r % 16, columns 8 q .. 8 q + 7
 *     (q = (c / 8) % 4) are the 16 bytes at element 8 * (16 q + r % 16).  Each block is then one
 *     v_mfma_f32_16x16x32_bf16 operand in lane order and a wave loads it as one contiguous
 *     kilobyte.  Buffers hold ceil(rows / 16) * 16 rows; rows past `rows` are never written.
 *     For an fp32 [rows, C] matrix (the decode residual stream x) the blocks are 16 x 32 floats
 *     (2 KB) in the same order, lane l = 16 q + r % 16 owning row r, columns 8 q .. 8 q + 7, its
 *     columns 0..3 at float 4 l and 4..7 at float 256 + 4 l of the block (two contiguous
 *     kilobytes per wave load).
 *   - KV cache layout is the reference StaticKVCache layout (src/inference.py:73-77):
 *     one layer's K (or V) is [batch, n_heads, cache_slots, 64] bf16, slot-major rows of 128 B.
 *     The fp32 form keeps the same layout in fp32 (rows of 256 B).
 *   - Two forms of the path.  A bf16 model (the reference's configurations 2-4) runs the bf16
 *     form: bf16 weights, bf16 q / K / V and cache.  A model with fp32 parameters runs the fp32
 *     form, as the reference keeps its cache and attention in the parameter dtype
 *     (src/inference.py:522, :544): each weight W passes as two bf16 matrices w = bf16(W) and
 *     w_lo = bf16(W - w) (the *_lo arguments of the K5 entries), q / K / V and the cache are
 *     fp32 (mdl_qkv_rope_cache with MDL_DTYPE_F32) and the attention is K4f (fp32 MFMA).
 */
#ifndef MDLARC_HIP_H
#define MDLARC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MDL_OK 0
#define MDL_ERR_NULL (-1)          /* a required pointer is NULL */
#define MDL_ERR_ALIGN (-2)         /* a pointer or leading dimension breaks 16-byte alignment */
#define MDL_ERR_SHAPE (-3)         /* a dimension is out of the supported range */
#define MDL_ERR_HEAD_DIM (-4)      /* head_dim != 64 or d_model != n_heads * 64 */
#define MDL_ERR_CACHE (-5)         /* slot range outside the cache */
#define MDL_ERR_WORKSPACE (-6)     /* workspace too small */
#define MDL_ERR_DTYPE (-7)         /* unsupported dtype code */
#define MDL_ERR_SCRATCH (-8)       /* work exceeds the library's static scratch buffer */

/* Size of the static device scratch buffer of mdl_attn_decode_rope_noalloc (per GPU). */
#define MDL_DECODE_SCRATCH_BYTES (4 << 20)

#define MDL_DTYPE_F32 0
#define MDL_DTYPE_BF16 1

/* Layout of a split activation written by a producer entry point (its *_layout argument). */
#define MDL_LAYOUT_ROWS 0          /* row-major [rows, 2K]: hi in columns [0, K), lo in [K, 2K) */
#define MDL_LAYOUT_TILES 1         /* the same matrix in MFMA tiles (see the conventions) */

/*
 * Soft decoding constraints on a row's logits, applied before the argmax in the order of
 * _apply_logit_constraints (src/inference.py:285-364; DecodingConstraints :37-43):
 *   1. logit v = -inf for every bit v set in disallow_mask (disallow_tokens);
 *   2. colours 0-9 with palette_mask[r*10 + c] == 0 lose palette_penalty;
 *   3. rows with a target shape (target_shape[r] = (h, w), both >= 0), grid state (x, y) =
 *      (grid_x[r], grid_y[r]) after the current token: x >= w -> colours lose shape_penalty;
 *      x < w -> NEWLINE loses it; y >= h -> colours and NEWLINE lose it (once more).
 * Each subtraction is a separate fp32 operation, as in the reference.  palette_mask and
 * target_shape may be NULL (that constraint is off); grid_x / grid_y are required with
 * target_shape.
 */
typedef struct mdl_logit_constraints {
  uint32_t disallow_mask;
  const uint8_t* palette_mask;  /* uint8 [rows, 10] */
  float palette_penalty;
  const int32_t* target_shape;  /* int32 [rows, 2] */
  const int32_t* grid_x;        /* int32 [rows] */
  const int32_t* grid_y;        /* int32 [rows] */
  float shape_penalty;
} mdl_logit_constraints;

/* Library version (major*100 + minor) and a static string for an error code. */
int mdl_version(void);
const char* mdl_error_string(int code);

/*
 * K1 -- token + example embedding gather fused with the first RMSNorm.
 * Replaces: TinyTransformer.forward token/example embedding (src/transformer.py:584-589),
 *           _prefill / _decode_step embedding (src/inference.py:393-395, :433-435),
 *           and the reduction of blocks[0].ln1 = RMSNorm.forward (src/transformer.py:45-48).
 * For row m (batch row b = m / row_len):
 *   x[m]     = tok_table[ids[m]] + (example_ids ? ex_table[example_ids[b]] : 0)     (fp32)
 *   rstd[m]  = 1 / sqrt(mean(x[m]^2) + eps)
 *   xs[m]    = split(x[m] * gamma)       bf16 [rows, 2d] (GEMM input; rstd is applied after
 *                                        the GEMM).  xs_out may be NULL.
 * layout: MDL_LAYOUT_ROWS, or MDL_LAYOUT_TILES (d a multiple of 32): x in the fp32 tile layout
 * and xs in the bf16 one, for the K5 decode entries.  xs_out and rstd_out may be NULL.
 * Tables are fp32 or bf16 (table_dtype); ids are clamped into range (callers validate first).
 */
int mdl_embed_rmsnorm(const int64_t* ids, const int64_t* example_ids, const void* tok_table,
                      const void* ex_table, int table_dtype, int vocab, int n_examples, int rows,
                      int row_len, int d, const float* gamma, float eps, float* x_out,
                      uint16_t* xs_out, float* rstd_out, int layout, void* stream);

/*
 * Decode-step entry: grid position of the token each row just emitted, then K1 on that token.
 * Replaces: GridStateUpdater.update (src/inference.py:127-168) followed by the embedding and
 *           blocks[0].ln1 of _decode_step (src/inference.py:433-437).
 * Per row b: pos_out[b] = position of token[b] from the state (gx, gy, in_out), the state
 * advances past it (the rule of mdl_grid_step), then x / xs / rstd as mdl_embed_rmsnorm with
 * row_len = 1 and layout as there (xs_out / rstd_out may be NULL).  counters (int32[2], may be
 * NULL) are incremented by one, as by mdl_grid_step.
 */
int mdl_decode_embed(const int64_t* token, const int64_t* example_ids, const void* tok_table,
                     const void* ex_table, int table_dtype, int vocab, int n_examples, int batch,
                     int d, const float* gamma, float eps, int32_t* gx, int32_t* gy,
                     uint8_t* in_out, int max_x, int max_y, int64_t* pos_out, int32_t* counters,
                     float* x_out, uint16_t* xs_out, float* rstd_out, int layout,
                     void* stream);

/*
 * Residual add fused with the next RMSNorm's reduction.
 * Replaces: the residual adds of TransformerBlock.forward (src/transformer.py:494-496),
 *           _prefill / _decode_step (src/inference.py:412-413, :455-456), the fc_down bias
 *           (src/transformer.py:443), and the reduction of the following ln2 / ln1 / ln_f.
 *   x[m]    += delta[m] (+ bias)           delta fp32 [rows, d] (may be NULL),
 *                                           bias fp32 [d] or NULL
 *   rstd[m]  = 1 / sqrt(mean(x[m]^2) + eps)
 *   xs[m]    = split(x[m] * gamma)         bf16 [rows, 2d] (skipped when xs_out is NULL), in
 *                                          xs_layout: MDL_LAYOUT_ROWS, or the bf16 tile layout
 *                                          (d a multiple of 16); x itself is row-major here
 */
int mdl_add_rmsnorm(float* x, const float* delta, const float* bias, int rows, int d,
                    const float* gamma, float eps, uint16_t* xs_out, float* rstd_out,
                    int xs_layout, void* stream);

/*
 * K2 -- RMSNorm scale + Q/K/V split + 3D RoPE + static-cache write.
 * Replaces: qkv reshape/unbind (src/inference.py:402-403, :439-440), the RMSNorm multiply of
 *           ln1, RotaryEmbedding3D.apply_rotary (src/transformer.py:132-187, _rotate_half
 *           :51-58), the transposes (src/inference.py:406) and StaticKVCache.update
 *           (src/inference.py:84-92).
 * qkv: fp32 [batch*seq, 3*d] (row stride qkv_ld elements) = (x*gamma) @ W_qkv^T, columns
 *      [q heads | k heads | v heads] (src/transformer.py:317-318).  rstd: fp32 [batch*seq].
 * pos: int64 [batch*seq, 3] (x, y, z); clamped to [0,max-1] per axis.
 * rope_tab: fp32 [cos_x(max_x*px) | sin_x | cos_y(max_y*py) | sin_y | cos_z(max_z*pz) | sin_z],
 *      the tables of RotaryEmbedding3D._build_cache (src/transformer.py:95-126).
 * Outputs: q_out [batch*seq, d] = rope(q * rstd) * q_scale; k/v written to cache slot
 *      (slot_dev ? *slot_dev : slot0) + s for token s of each batch row.  For the attention
 *      kernels (K4a, K4b, K4f) q_scale is the softmax scale times log2(e): their softmax is
 *      base 2.  out_dtype (MDL_DTYPE_BF16 or MDL_DTYPE_F32) is the type of q_out and of the
 *      cache: bf16 for the bf16 form, fp32 for the fp32 form (then nothing is rounded).
 */
int mdl_qkv_rope_cache(const float* qkv, int64_t qkv_ld, const float* rstd,
                       const int64_t* pos, const float* rope_tab, int batch, int seq,
                       int n_heads, int head_dim, int max_x, int max_y, int max_z, int px,
                       int py, int pz, float q_scale, void* q_out, void* k_cache,
                       void* v_cache, int out_dtype, int cache_slots, int slot0,
                       const int32_t* slot_dev, void* stream);

/*
 * K2 over a packed token list (the prompt tokens of every row without their left padding).
 * Replaces: the same reference ops as mdl_qkv_rope_cache over the rows of a left-padded batch,
 *           for the tokens at or after each row's first valid position (src/inference.py:395-407;
 *           the padding's K/V are never visible to a later query).
 * qkv / rstd / pos / q_out hold n_tokens rows.  Token m belongs to batch row token_row[m] and
 * writes its k / v into cache slot token_slot[m] of that row (nothing when token_slot[m] < 0,
 * or outside [0, cache_slots) or a token_row outside [0, batch)).  out_dtype as for
 * mdl_qkv_rope_cache.
 */
int mdl_qkv_rope_cache_packed(const float* qkv, int64_t qkv_ld, const float* rstd,
                              const int64_t* pos, const float* rope_tab, int64_t n_tokens,
                              const int32_t* token_row, const int32_t* token_slot, int batch,
                              int n_heads, int head_dim, int max_x, int max_y, int max_z, int px,
                              int py, int pz, float q_scale, void* q_out, void* k_cache,
                              void* v_cache, int out_dtype, int cache_slots, void* stream);

/*
 * K3 -- SwiGLU gate: silu(gate) * up, with the RMSNorm multiply of ln2 and the fc biases.
 * Replaces: FeedForward.forward's silu(fc_gate(x)) * fc_up(x) (src/transformer.py:441-449).
 * gate_up: fp32 [rows, 2*d_ff] (row stride ld) = (x*gamma2) @ [W_gate; W_up]^T.
 *   h[m, j] = silu(rstd[m]*g[m,j] + bias_gate[j]) * (rstd[m]*u[m,j] + bias_up[j])
 * h_out: split bf16 [rows, 2*d_ff] in h_layout (MDL_LAYOUT_TILES needs d_ff % 16 == 0).
 * rstd / biases may be NULL (treated as 1 / 0).  d_ff must be a multiple of 8.
 */
int mdl_swiglu(const float* gate_up, int64_t ld, const float* rstd, const float* bias_gate,
               const float* bias_up, int rows, int d_ff, uint16_t* h_out, int h_layout,
               void* stream);

/*
 * The three fused kernels in the format of BASELINE's fused-kernel microbench (bf16
 * activations in and out, no split outputs): the reference's bf16 model keeps its activations
 * in bf16 (model.to(bfloat16), src/inference.py:522, :544).  The inference path above keeps
 * fp32 GEMM outputs and split GEMM inputs instead (they hold the logits within the fp32
 * reference's tolerance); these entries serve bf16-activation pipelines.
 */

/*
 * K1, bf16 form.  Replaces: token_embed(ids) + example_embed(example_ids) and ln1
 * (src/transformer.py:584-589, RMSNorm :37-48) for a bf16 model.
 * tok_table / ex_table bf16 [vocab, d] / [n_examples, d]; example_ids as mdl_embed_rmsnorm
 * (may be NULL).  x_out = bf16(tok + ex) and xn_out = bf16(x * rstd * gamma), rstd from the
 * rounded x; both bf16 [rows, d] row-major.  d a multiple of 8, at most 2048.
 */
int mdl_embed_rmsnorm_bf16(const int64_t* ids, const int64_t* example_ids,
                           const uint16_t* tok_table, const uint16_t* ex_table, int vocab,
                           int n_examples, int rows, int row_len, int d, const float* gamma,
                           float eps, uint16_t* x_out, uint16_t* xn_out, void* stream);

/*
 * K2, bf16 form: mdl_qkv_rope_cache on a bf16 qkv row (the output of a bf16 projection),
 * rstd may be NULL (qkv already normed).  Same outputs, positions, cache slots and rounding.
 * Replaces: the qkv split, RotaryEmbedding3D.apply_rotary and StaticKVCache.update
 * (src/transformer.py:132-187, src/inference.py:84-92) for a bf16 model.  n_heads in
 * {4, 12, 16, 20} (the reference presets).
 */
int mdl_qkv_rope_cache_bf16(const uint16_t* qkv, int64_t qkv_ld, const float* rstd,
                            const int64_t* pos, const float* rope_tab, int batch, int seq,
                            int n_heads, int head_dim, int max_x, int max_y, int max_z, int px,
                            int py, int pz, float q_scale, uint16_t* q_out, uint16_t* k_cache,
                            uint16_t* v_cache, int cache_slots, int slot0, void* stream);

/*
 * K3, bf16 form: gate_up bf16 [rows, 2*d_ff] (row stride ld, a multiple of 8) in, h_out bf16
 * [rows, d_ff] = bf16(silu(rstd*g + b_g) * (rstd*u + b_u)) out.  rstd / biases may be NULL.
 * Replaces: FeedForward.forward's silu(fc_gate(x)) * fc_up(x) (src/transformer.py:441-449)
 * for a bf16 model.
 */
int mdl_swiglu_bf16(const uint16_t* gate_up, int64_t ld, const float* rstd,
                    const float* bias_gate, const float* bias_up, int rows, int d_ff,
                    uint16_t* h_out, void* stream);

/*
 * K5 -- decode projection GEMM on split activations (bf16 MFMA, fp32 accumulation).
 * Replaces: the nn.Linear projections of one decode step -- qkv_proj (src/inference.py:439),
 *           out_proj (:453), fc_gate / fc_up and fc_down (FeedForward.forward,
 *           src/transformer.py:441-449) -- at decode-sized row counts.
 *   out[i, j] (fp32, row stride ldo) = sum_{k < K} (a[i, k] + a[i, K + k]) * w[j, k]
 * a: split bf16 activation [m, 2K] (hi in columns [0, K), lo in [K, 2K)) in a_layout; w: bf16
 * [n, K] in nn.Linear orientation in w_layout.  A row-major operand has row stride lda / ldw
 * (the left half of a [W | W] operand serves, ldw = 2K); a tiled one (MDL_LAYOUT_TILES, from the
 * producers' *_layout argument or mdl_tile_matrix) ignores its ld.  Both tiled is the fast form
 * (contiguous kilobyte loads).  k must be a positive multiple of 32 and n a multiple of 4;
 * pointers 16-byte aligned, row-major lda / ldw multiples of 8, ldo a multiple of 4.
 * tile = 0 picks the block shape from (m, n, k) (mdl_gemm_split_pick); 1 .. mdl_gemm_split_tiles()
 * forces one.  A given tile gives bit-identical results run to run and across layouts; tiles
 * differ at fp32 rounding.
 */
int mdl_gemm_split(const uint16_t* a, int64_t lda, int a_layout, const uint16_t* w, int64_t ldw,
                   int w_layout, float* out, int64_t ldo, int m, int n, int k, int tile,
                   void* stream);
/*
 * K5 with the SwiGLU gate (K3) fused into its epilogue, for the decode step:
 *   h[i, c] = silu(rstd[i] g + bias_gate[c]) * (rstd[i] u + bias_up[c]),
 *   g, u = the fc_gate / fc_up rows c of w_gu against a, as mdl_gemm_split computes them,
 * written as the split h of mdl_swiglu ([m, 2 d_ff], MDL_LAYOUT_TILES) with no fp32 gate / up
 * round trip; the result equals mdl_gemm_split + mdl_swiglu bit for bit for the same tile.
 * Replaces: FeedForward.forward's silu(fc_gate(x)) * fc_up(x) (src/transformer.py:441-449).
 * a: split activation [m, 2k] in MDL_LAYOUT_TILES.  w_gu: [W_gate; W_up] ([2 d_ff, k]) with
 * their 16-row blocks interleaved (row block 2 b = W_gate rows 16 b .. 16 b + 15, row block
 * 2 b + 1 = W_up rows 16 b ..), in MDL_LAYOUT_TILES.  rstd / biases may be NULL (1 / 0).
 * d_ff a multiple of 16, k of 32; tile as for mdl_gemm_split (chosen for n = 2 d_ff).
 */
int mdl_gemm_split_swiglu(const uint16_t* a, const uint16_t* w_gu, const float* rstd,
                          const float* bias_gate, const float* bias_up, uint16_t* h_out, int m,
                          int d_ff, int k, int tile, void* stream);
/*
 * K5 with the RMSNorm of the projection's input fused into its prologue (decode step):
 *   out[i, j] = sum_k split(x[i, k] * gamma[k]) * w[j, k]       (fp32, row stride ldo)
 *   rstd_out[i] = 1 / sqrt(mean_k(x[i, k]^2) + eps)              (may be NULL)
 * x: the fp32 residual stream [m, k] in MDL_LAYOUT_TILES (written by mdl_decode_embed /
 * mdl_embed_rmsnorm with that layout and updated by mdl_gemm_split_residual); w tiled [n, k].
 * split(x * gamma) and rstd are what mdl_add_rmsnorm would write (rstd to fp32 rounding: the
 * sum of squares is taken in another order), so this replaces that launch and the split
 * activation buffer.  k a positive multiple of 32, n of 16.
 * w_lo (may be NULL): the low bf16 part of an fp32 weight (w_lo = bf16(W - w), tiled like w);
 * each k-step then also adds split_hi . w_lo, so the product sees W to ~2^-17 (the fp32 form).
 * Any m: the fp32 form also runs a prompt's projections here.
 * Replaces: qkv_proj(ln1(x)) (src/inference.py:438-439; RMSNorm.forward
 *           src/transformer.py:45-48).
 */
int mdl_gemm_norm(const float* x, const float* gamma, float eps, const uint16_t* w,
                  const uint16_t* w_lo, float* out, int64_t ldo, float* rstd_out, int m, int n,
                  int k, int tile, void* stream);
/*
 * mdl_gemm_norm with K2 in its epilogue, for the decode step: from qkv = split(x * gamma) . w^T
 * (w: qkv_proj tiled [3 d, d], d = n_heads * 64) and rstd it writes exactly what
 * mdl_qkv_rope_cache writes for one token per row (the same arithmetic): q_out bf16 [m, d]
 * (RoPE, q_scale) and K / V into slot t = *slot_dev (or slot0) of cache row m
 * ([m, n_heads, cache_slots, 64]); rstd_out may be NULL.  The attention then runs unfused
 * (mdl_attn_decode on q_out).  tile as for mdl_gemm_norm.
 * Replaces: qkv_proj(ln1(x)), the q / k / v split, RotaryEmbedding3D and the cache write of
 *           _decode_step (src/inference.py:437-445; src/transformer.py:132-187, :248-263).
 */
int mdl_gemm_norm_qkv(const float* x, const float* gamma, float eps, const uint16_t* w, int m,
                      int n_heads, float* rstd_out, const int64_t* pos, const float* rope_tab,
                      int max_x, int max_y, int max_z, int px, int py, int pz, float q_scale,
                      uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, int cache_slots,
                      int slot0, const int32_t* slot_dev, int tile, void* stream);
/*
 * mdl_gemm_norm feeding the SwiGLU epilogue of mdl_gemm_split_swiglu (rstd from the prologue):
 * h = split(silu(rstd g + bias_gate) * (rstd u + bias_up)) with g / u the gate / up rows of
 * w_gu against split(x * gamma).  w_gu_lo (may be NULL): the low part of an fp32 w_gu, as
 * w_lo of mdl_gemm_norm.  Replaces ffn(ln2(x))'s gate (src/transformer.py:441-449, :494-496).
 */
int mdl_gemm_norm_swiglu(const float* x, const float* gamma, float eps, const uint16_t* w_gu,
                         const uint16_t* w_gu_lo, const float* bias_gate, const float* bias_up,
                         uint16_t* h_out, int m, int d_ff, int k, int tile, void* stream);
/*
 * K5 with the residual add in its epilogue (decode step): x[i, j] += sum_k (a_hi + a_lo)[i, k]
 * w[j, k] (+ bias[j]), in place on the fp32 residual stream x [m, n] in MDL_LAYOUT_TILES; a the
 * tiled split activation [m, 2k], w tiled [n, k], bias [n] or NULL.  n a multiple of 32.
 * w_lo (may be NULL): the low part of an fp32 w, as for mdl_gemm_norm.
 * Replaces: the residual adds x + out_proj(...) and x + fc_down(...) (+ its bias) of
 *           _decode_step (src/inference.py:453-456; src/transformer.py:443, :494-496).
 */
int mdl_gemm_split_residual(const uint16_t* a, const uint16_t* w, const uint16_t* w_lo, float* x,
                            const float* bias, int m, int n, int k, int tile, void* stream);
/* Number of compiled block shapes, and the automatic choice for (m, n, k) of the split forms
 * (host only; the norm forms weight the activation rows twice, see csrc/split_gemm.hip). */
int mdl_gemm_split_tiles(void);
int mdl_gemm_split_pick(int m, int n, int k);
/*
 * K6 -- the projections of a prompt (prefill, forward): the K5 formulations at prompt-sized
 * row counts, in 256 x 256 output tiles through LDS.  Weights are the tiled copies K5 uses
 * (w: [n, k] MDL_LAYOUT_TILES; w_gu: interleaved gate / up, tiled).  Results are reproducible
 * run to run; they differ from K5 and from hipBLASLt at fp32 rounding (another summation
 * order).  k a positive multiple of 32, n (and 2 d_ff) of 16; pointers 16-byte aligned.
 * Replaces: qkv_proj / out_proj (src/transformer.py:248-263) and fc_gate / fc_up / fc_down
 *           (FeedForward.forward, :441-449) over a prompt (TinyTransformer.forward
 *           :562-599, _prefill src/inference.py:383-424), with the RMSNorms (:45-48) and the
 *           residual adds (TransformerBlock.forward :486-497) fused in.
 *
 * a_parts (the split forms and the SwiGLU form): 2 -- the activation is split, hi and lo, as
 * everywhere else; 1 -- the lo term is dropped: a holds hi alone ([m, k]; row stride lda >= k
 * when row-major), and the norm form uses bf16(x * gamma).  Half the MFMA work; the products
 * then carry the activation's bf16 rounding (2^-9 relative) instead of ~2^-17.
 *
 * mdl_prefill_gemm_split:   out[i, j] = sum_k (a_hi + a_lo)[i, k] w[j, k] (fp32, row stride
 *                           ldo); a split [m, a_parts k] in a_layout (row stride lda when
 *                           row-major).
 * mdl_prefill_gemm_norm:    out = split(x * gamma) . w^T and rstd_out[i] (may be NULL) =
 *                           1 / sqrt(mean_k x[i, k]^2 + eps), x the fp32 residual stream [m, k]
 *                           in MDL_LAYOUT_TILES: the ln1 + qkv_proj pair with rstd deferred to
 *                           the consumer (as mdl_gemm_norm); k at most 2048.
 * mdl_prefill_gemm_norm_swiglu: h = split(silu(rstd g + bias_gate) * (rstd u + bias_up)), g / u
 *                           the gate / up rows of w_gu against split(x * gamma) (x as above);
 *                           h_out tiled [m, h_parts d_ff] (ceil(m / 16) * 16 rows): hi, then lo
 *                           when h_parts is 2 (h_parts 1 feeds a consumer with a_parts 1);
 *                           biases may be NULL.
 * mdl_prefill_gemm_split_residual: x[i, j] += sum_k (a_hi + a_lo)[i, k] w[j, k] (+ bias[j]) in
 *                           place, x the fp32 residual stream [m, n] in MDL_LAYOUT_TILES (n a
 *                           multiple of 32); bias may be NULL.
 * a_parts or h_parts other than 1 or 2: MDL_ERR_SHAPE.
 */
int mdl_prefill_gemm_split(const uint16_t* a, int64_t lda, int a_layout, int a_parts,
                           const uint16_t* w, float* out, int64_t ldo, int m, int n, int k,
                           void* stream);
int mdl_prefill_gemm_norm(const float* x, const float* gamma, float eps, const uint16_t* w,
                          float* out, int64_t ldo, float* rstd_out, int m, int n, int k,
                          void* stream);
int mdl_prefill_gemm_norm_swiglu(const float* x, const float* gamma, float eps, int a_parts,
                                 const uint16_t* w_gu, const float* bias_gate,
                                 const float* bias_up, uint16_t* h_out, int h_parts, int m,
                                 int d_ff, int k, void* stream);
int mdl_prefill_gemm_split_residual(const uint16_t* a, int64_t lda, int a_layout, int a_parts,
                                    const uint16_t* w, float* x, const float* bias, int m, int n,
                                    int k, void* stream);
/*
 * K6 with K2 (mdl_qkv_rope_cache) in its epilogue: ln1 + qkv_proj + RoPE + cache write of a
 * prompt in one launch.  w: qkv_proj tiled [3 d, d] (d = n_heads * 64, at most 2048); x as for
 * mdl_prefill_gemm_norm.  Writes, from the projection's fp32 accumulators and rstd, exactly what
 * mdl_qkv_rope_cache(_packed) writes (the same arithmetic): q_out bf16 [m, d] (RoPE, q_scale),
 * K / V into one layer's cache [batch, n_heads, cache_slots, 64]; rstd_out [m] (may be NULL);
 * and the fp32 accumulators of the lead rows -- token slots kv_start[b] .. kv_start[b] + lead - 1
 * of each batch row (kv_start may be NULL: 0) -- into qkv_lead (row stride ldq, may be NULL), the
 * rows mdl_attn_prefill_lead reads.  Rows: a packed token list (token_row / token_slot, both or
 * neither; a negative slot writes no K / V), or [batch, seq] (m = batch * seq, token i of row b
 * in slot i).  Rope arguments as for mdl_qkv_rope_cache.
 * Replaces: qkv_proj(ln1(x)) and the q / k / v split, RotaryEmbedding3D and the cache write of
 *           _prefill / Attention.forward (src/inference.py:396-407; src/transformer.py:248-263,
 *           :132-187).
 */
int mdl_prefill_gemm_norm_qkv(const float* x, const float* gamma, float eps, const uint16_t* w,
                              int m, int n_heads, float* rstd_out, float* qkv_lead, int64_t ldq,
                              int lead, const int32_t* kv_start, const int64_t* pos,
                              const float* rope_tab, int max_x, int max_y, int max_z, int px,
                              int py, int pz, float q_scale, uint16_t* q_out, uint16_t* k_cache,
                              uint16_t* v_cache, int cache_slots, int batch, int seq,
                              const int32_t* token_row, const int32_t* token_slot, void* stream);
/*
 * dst = src ([rows, cols] bf16, row stride ld) in MDL_LAYOUT_TILES, rows padded to a multiple
 * of 16 with zeros (dst holds ceil(rows / 16) * 16 * cols elements).  cols a multiple of 32.
 * Packs the decode weights once per model version (no reference counterpart: a layout step).
 */
int mdl_tile_matrix(const uint16_t* src, int64_t ld, int rows, int cols, uint16_t* dst,
                    void* stream);

/*
 * K4a -- prefill / full-sequence attention on bf16 MFMA (flash style, online softmax).
 * Replaces: F.scaled_dot_product_attention in _prefill (src/inference.py:409, mask from
 *           _build_sdpa_mask :372-380, is_causal=True) and in MultiHeadSelfAttention.forward
 *           (src/transformer.py:333-349, is_causal either way).
 * q: bf16 [batch, seq, n_heads, 64], already multiplied by the softmax scale and by log2(e)
 *    (the kernel's softmax is base 2: p = 2^(q.k - max)).
 * out: split bf16 [batch*seq, 2*n_heads*64] (the out-projection GEMM input) in out_layout
 *      (MDL_LAYOUT_ROWS, or MDL_LAYOUT_TILES with rows padded to a multiple of 16).
 * keys:    k_cache / v_cache slots [0, seq) of [batch, n_heads, cache_slots, 64].
 * Query i of row b sees key j iff j < seq, key_mask[b*seq + j] != 0 (key_mask may be NULL),
 * j >= kv_start[b] (kv_start may be NULL; it must not exclude a visible key) and, if causal,
 * j <= i.  A query with no visible key outputs 0 (torch CPU SDPA semantics).
 * row_holes (uint8 [batch], may be NULL): 0 promises that row b's key mask is set exactly on
 *   [kv_start[b], seq), so the kernel skips reading it (mdl_grid_init computes it).
 */
int mdl_attn_prefill(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                     int batch, int seq, int n_heads, int head_dim, int cache_slots,
                     const uint8_t* key_mask, const uint8_t* row_holes, const int32_t* kv_start,
                     int causal, uint16_t* out, int out_layout, void* stream);

/*
 * K4a over packed query rows: as mdl_attn_prefill, for the queries i >= kv_start[b] of each row
 * only.  Query i of row b is row q_offset[b] + i - kv_start[b] of q (bf16 [rows, n_heads, 64])
 * and of out (split bf16 [rows, 2*n_heads*64], in out_layout); no other row of out is
 * written.  Keys are the
 * cache slots as in mdl_attn_prefill; slots before kv_start[b] are never read into a product.
 * kv_start and q_offset are required; the caller sizes q / out to cover every row it names.
 * Replaces: the same SDPA call as mdl_attn_prefill (src/inference.py:409), without the padding
 *           queries: each sees no key, so its output is 0, which the caller supplies if needed.
 */
int mdl_attn_prefill_packed(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                            int batch, int seq, int n_heads, int head_dim, int cache_slots,
                            const uint8_t* key_mask, const uint8_t* row_holes,
                            const int32_t* kv_start, const int32_t* q_offset, int causal,
                            uint16_t* out, int out_layout, void* stream);

/*
 * K4c -- exact (fp32) causal attention for the lead queries of each row, after K4a.
 * Replaces: the same SDPA call as mdl_attn_prefill (src/inference.py:409; src/transformer.py:
 *           333-349 with is_causal=True) for the first 64 queries at or after kv_start[b]: those
 *           see at most 64 keys, so K4a's bf16 roundings of q, K, V and the probabilities are
 *           not averaged away there.
 * qkv / rstd / pos: the projection GEMM's fp32 output and the inputs K2 consumed
 *   (mdl_qkv_rope_cache, same layout and rope arguments).  q_scale is the softmax scale itself
 *   (this pass computes its softmax in fp32 with natural exponentials).  Token position i
 *   of row b is row b*seq + i of them and of out, or, with q_offset (packed rows; kv_start then
 *   required), row q_offset[b] + i - kv_start[b].
 * Recomputes q, k, v of those tokens in fp32 (RMSNorm scale, 3D RoPE, softmax scale), applies
 * the key mask as mdl_attn_prefill does and overwrites the split output rows of the first
 * min(64, seq - kv_start[b]) queries (out in out_layout, as K4a wrote it); every other row of
 * out is left as it is.
 */
int mdl_attn_prefill_lead(const float* qkv, int64_t qkv_ld, const float* rstd,
                          const int64_t* pos, const float* rope_tab, int max_x, int max_y,
                          int max_z, int px, int py, int pz, float q_scale, int batch, int seq,
                          int n_heads, int head_dim, const uint8_t* key_mask,
                          const int32_t* kv_start, const int32_t* q_offset, uint16_t* out,
                          int out_layout, void* stream);

/*
 * K4b -- decode attention over the static cache (split-K flash decoding on bf16 MFMA: QK^T with
 * K straight from HBM as the A operand, PV with V staged through LDS; the probabilities enter
 * the PV product rounded to bf16).
 * Replaces: F.scaled_dot_product_attention in _decode_step (src/inference.py:452) with the
 *           mask rebuilt from full_attention_mask (src/inference.py:446-450, :557-558, :626).
 * q: bf16 [batch, n_heads, 64], pre-scaled as for mdl_attn_prefill (softmax scale times
 *    log2(e)); out: split bf16 [batch, 2*n_heads*64] in
 * out_layout (MDL_LAYOUT_ROWS or MDL_LAYOUT_TILES).
 * The query of row b sees slot j iff
 *   kv_start[b] <= j <= t, t = (seq_dev ? *seq_dev : seq_pos), and
 *   (j >= prompt_len || prompt_mask[b*prompt_len + j] != 0)   (prompt_mask may be NULL).
 * row_holes (uint8 [batch], may be NULL): 0 promises that row b's prompt mask is set exactly
 *   on [kv_start[b], prompt_len), so the kernel skips reading it (mdl_grid_init computes it).
 * row_order (int32 [batch], may be NULL): a permutation of the rows giving the order their work
 *   is dispatched in; longest-first (ascending kv_start) shortens the launch's tail.
 * workspace: fp32, at least mdl_attn_decode_workspace_bytes(...) bytes (may be NULL when
 *   that is 0).  split_len: slots per work item (multiple of 128, >= 128; mdl_attn_decode_f32
 *   takes multiples of 16 and the same workspace size).
 */
int64_t mdl_attn_decode_workspace_bytes(int batch, int n_heads, int cache_slots, int split_len);
int mdl_attn_decode(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                    int batch, int n_heads, int head_dim, int cache_slots,
                    const uint8_t* prompt_mask, int prompt_len, const uint8_t* row_holes,
                    const int32_t* kv_start, const int32_t* row_order, int seq_pos,
                    const int32_t* seq_dev,
                    float* workspace, int64_t workspace_bytes, int split_len, uint16_t* out,
                    int out_layout, void* stream);

/*
 * K2 + K4b fused for the decode step: mdl_qkv_rope_cache (seq = 1, slot t) followed by
 * mdl_attn_decode, in one launch.  Each (row, head) block rotates its head's q and k of the
 * decode token from qkv (fp32 [batch, 3*d], row stride qkv_ld), writes k / v into cache slot t
 * (t = seq_dev ? *seq_dev : seq_pos) and attends as mdl_attn_decode.  q is rounded to bf16 as
 * mdl_qkv_rope_cache rounds it.  Arguments as in those two entry points.
 * Replaces: the same reference ops as mdl_qkv_rope_cache and mdl_attn_decode, for one token.
 */
int mdl_attn_decode_rope(const float* qkv, int64_t qkv_ld, const float* rstd, const int64_t* pos,
                         const float* rope_tab, int max_x, int max_y, int max_z, int px, int py,
                         int pz, float q_scale, uint16_t* k_cache, uint16_t* v_cache, int batch,
                         int n_heads, int head_dim, int cache_slots, const uint8_t* prompt_mask,
                         int prompt_len, const uint8_t* row_holes, const int32_t* kv_start,
                         const int32_t* row_order, int seq_pos, const int32_t* seq_dev,
                         float* workspace, int64_t workspace_bytes, int split_len, uint16_t* out,
                         int out_layout, void* stream);

/*
 * mdl_attn_decode_rope without the workspace argument: the split partials go to a static
 * device array of MDL_DECODE_SCRATCH_BYTES (4 MiB) per GPU instead, so the call allocates
 * nothing, on the host or the device, and asks its caller for no buffer beyond the inputs and
 * outputs.  No counterpart in the reference: it is for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Work needing more than MDL_DECODE_SCRATCH_BYTES (mdl_attn_decode_workspace_bytes of the same
 * arguments) returns MDL_ERR_SCRATCH before any launch.  The device address of the array is
 * looked up (hipGetSymbolAddress) on the first call on each device; make that first call
 * outside graph capture.  Every call on one GPU shares its array: calls that overlap in time on
 * one GPU (two streams, two threads) race and must be ordered by the caller.  Nothing in the
 * array needs clearing between calls: each split writes its whole partial before it is read.
 * Other arguments and results as mdl_attn_decode_rope.
 */
int mdl_attn_decode_rope_noalloc(const float* qkv, int64_t qkv_ld, const float* rstd,
                                 const int64_t* pos, const float* rope_tab, int max_x, int max_y,
                                 int max_z, int px, int py, int pz, float q_scale,
                                 uint16_t* k_cache, uint16_t* v_cache, int batch, int n_heads,
                                 int head_dim, int cache_slots, const uint8_t* prompt_mask,
                                 int prompt_len, const uint8_t* row_holes,
                                 const int32_t* kv_start, const int32_t* row_order, int seq_pos,
                                 const int32_t* seq_dev, int split_len, uint16_t* out,
                                 int out_layout, void* stream);

/*
 * K4f -- attention of the fp32 form over an fp32 cache, on fp32 MFMA: the operands enter the
 * products unrounded and the softmax stays fp32; only the output is stored, as the split
 * (hi|lo bf16) input of the out projection.
 * Replaces: F.scaled_dot_product_attention of _prefill (src/inference.py:409) and of
 *           TinyTransformer.forward (src/transformer.py:333-349) for a model whose parameters
 *           (and so its cache, src/inference.py:522, :544) are fp32.
 * q: fp32 [rows, n_heads, 64], pre-scaled by the softmax scale times log2(e) (mdl_qkv_rope_cache
 *    with MDL_DTYPE_F32); k_cache / v_cache: fp32 [batch, n_heads, cache_slots, 64], keys in
 *    slots [0, seq).
 * Query i of row b sees key j iff j < seq, kv_start[b] <= j (kv_start may be NULL), key_mask[b *
 * seq + j] != 0 (key_mask may be NULL) and, if causal, j <= i; a query with no visible key
 * outputs 0.  Query rows: b * seq + i, or with q_offset (packed rows; kv_start then required)
 * row q_offset[b] + i - kv_start[b] for the queries i >= kv_start[b] only.
 * out: split bf16 [rows, 2 * n_heads * 64] in out_layout; rows not named are not written.
 */
int mdl_attn_prefill_f32(const float* q, const float* k_cache, const float* v_cache, int batch,
                         int seq, int n_heads, int head_dim, int cache_slots,
                         const uint8_t* key_mask, const int32_t* kv_start,
                         const int32_t* q_offset, int causal, uint16_t* out, int out_layout,
                         void* stream);

/*
 * K4f at decode: the query of row b (q row b) sees slot j iff kv_start[b] <= j <= t,
 * t = (seq_dev ? *seq_dev : seq_pos), and (j >= prompt_len || prompt_mask[b * prompt_len + j]
 * != 0) (prompt_mask may be NULL) -- the visibility rule of mdl_attn_decode.  K / V of slot t
 * must be written first (mdl_qkv_rope_cache, seq = 1, slot_dev).  The slots of a row are split
 * into chunks of split_len (a positive multiple of 16), one wave each; with more than one chunk
 * (cache_slots > split_len) the chunks' states go to `workspace`, which must hold
 * mdl_attn_decode_workspace_bytes(batch, n_heads, cache_slots, split_len) bytes (16-byte
 * aligned; else MDL_ERR_WORKSPACE), and a second launch merges them.  Arguments otherwise as for
 * mdl_attn_prefill_f32.
 * Replaces: F.scaled_dot_product_attention in _decode_step (src/inference.py:452) for an fp32
 *           model, with the mask of src/inference.py:446-450.
 */
int mdl_attn_decode_f32(const float* q, const float* k_cache, const float* v_cache, int batch,
                        int n_heads, int head_dim, int cache_slots, const uint8_t* prompt_mask,
                        int prompt_len, const int32_t* kv_start, int seq_pos,
                        const int32_t* seq_dev, float* workspace, int64_t workspace_bytes,
                        int split_len, uint16_t* out, int out_layout, void* stream);

/*
 * Final RMSNorm + LM head + greedy argmax.
 * Replaces: model.lm_head(model.ln_f(x)) in _prefill / _decode_step (src/inference.py:417-424,
 *           :459) including the x[b, lengths-1] row pick, and logits.argmax(-1)
 *           (src/inference.py:573-574, :610-611; first index on ties).
 * Row r uses x[row_index ? row_index[r] : r].  logits_out fp32 [rows, vocab] and token_out
 * int64 [rows] may each be NULL.  w_head fp32 [vocab, d], gamma fp32 [d].  vocab <= 32.
 * constraints (may be NULL) are applied to row r's logits before the argmax; logits_out then
 * holds the constrained logits.  x_layout: MDL_LAYOUT_ROWS, or MDL_LAYOUT_TILES (the fp32 tile
 * layout of the decode residual stream; d a multiple of 32).
 */
int mdl_lm_head(const float* x, const int32_t* row_index, int rows, int d, const float* gamma,
                float eps, const float* w_head, int vocab, float* logits_out, int64_t* token_out,
                const mdl_logit_constraints* constraints, int x_layout, void* stream);

/*
 * Decode-step tail: final RMSNorm + LM head + greedy argmax + token commit in one launch.
 * Replaces: lm_head(ln_f(x)) and argmax of _decode_step / generate_output
 *           (src/inference.py:459, :610-611), generated.append and finished |= END
 *           (src/inference.py:589-590, :622-626).
 * token_out[b] = argmax; out_ids[b*out_ld + c] = token_out[b] with c = (counters ? counters[1]
 * : col); finish_step[b] (may be NULL) = c - gen_base at the first END.  logits_out may be NULL.
 * constraints (may be NULL) as for mdl_lm_head, with the grid state the step's mdl_decode_embed
 * advanced (so constrained greedy decoding replays from a captured graph too).  x_layout as
 * for mdl_lm_head.
 */
int mdl_decode_head(const float* x, int batch, int d, const float* gamma, float eps,
                    const float* w_head, int vocab, float* logits_out, int64_t* token_out,
                    int64_t* out_ids, int64_t out_ld, int col, const int32_t* counters,
                    int32_t* finish_step, int gen_base, int end_id,
                    const mdl_logit_constraints* constraints, int x_layout,
                    void* stream);

/*
 * Grid-state initialisation from the prompt.
 * Replaces: _derive_initial_state_from_prompt (src/inference.py:171-221) and the
 *           lengths-1 index of _prefill (src/inference.py:420-424).
 * ids int64 [batch, seq], pos int64 [batch, seq, 3], mask uint8 [batch, seq] or NULL (all valid).
 * row_shift int32 [batch] or NULL (all 0): for rows that the reference would have left-padded in
 *   a narrower batch of width L, the extra left padding seq - L of this batch; the reference's
 *   index len-1 in its own batch is index row_shift[b] + len-1 here (clamped into the row).
 *   Several such batches (the reference's chunks of 16) then run as one with identical results.
 * Outputs per row: gx, gy (int32), in_out (uint8), kv_start = first valid index (seq if none),
 * last_row = b*seq + row_shift[b] + max(len-1, 0) (the row the reference's prefill reads its
 * logits from; the grid state derives from the same token), row_holes = 1 if the valid positions
 * are not the single run [kv_start, seq), else 0.  kv_start / last_row / row_holes may each be
 * NULL.
 */
int mdl_grid_init(const int64_t* ids, const int64_t* pos, const uint8_t* mask,
                  const int32_t* row_shift, int batch, int seq, int max_x, int max_y, int32_t* gx,
                  int32_t* gy, uint8_t* in_out, int32_t* kv_start, int32_t* last_row,
                  uint8_t* row_holes, void* stream);

/*
 * Augmented prompts of one task, built on the device and left-padded into one batch.
 * Replaces: the prompt construction of _predict_augmentations_batched (src/inference.py:794-827,
 *           :877-890): dihedral transforms (src/data.py:224-233), colour permutations (:257-278),
 *           encode_example (:75-93), compute_positions_3d (:124-175) and the END / (0,0,0) left
 *           padding.
 * cells uint8 [n_cells]: every grid of the task row-major in its own orientation, concatenated;
 * grids int32 [n_grids, 3] = (offset into cells, h, w) in the order in0, out0, in1, out1, ...,
 *   test_in (n_grids odd);
 * variants int32 [batch, 2] = (dihedral index 0-7, row of perms); perms int32 [n_perms, 10];
 * lengths int32 [batch]: each variant's prompt length (sum of its grids' h'(w'+1) plus the
 *   START / IO_SEP / END tokens), seq >= max(lengths).
 * Outputs: ids int64 [batch, seq], pos int64 [batch, seq, 3], mask uint8 [batch, seq]; row b's
 * prompt occupies columns [seq - lengths[b], seq).
 */
int mdl_build_prompts(const uint8_t* cells, int64_t n_cells, const int32_t* grids, int n_grids,
                      const int32_t* variants, int batch, const int32_t* perms, int n_perms,
                      const int32_t* lengths, int seq, int64_t* ids_out, int64_t* pos_out,
                      uint8_t* mask_out, void* stream);

/*
 * One grid-state step: position of the token each row just emitted, then advance the state.
 * Replaces: GridStateUpdater.update (src/inference.py:127-168).
 * token int64 [batch] -> pos_out int64 [batch, 3].  counters (int32[2], may be NULL) are
 * incremented by one by this launch: {cache slot of the current token, output column}.
 */
int mdl_grid_step(const int64_t* token, int batch, int max_x, int max_y, int32_t* gx,
                  int32_t* gy, uint8_t* in_out, int64_t* pos_out, int32_t* counters,
                  void* stream);

/*
 * Commit one generated token per row.
 * Replaces: generated.append / finished |= (next_token == END) (src/inference.py:589-590,
 *           :622-626).
 * out_ids[b*out_ld + c] = token[b], c = (counters ? counters[1] : col).  If token[b] == end_id
 * and finish_step[b] < 0, finish_step[b] = c - gen_base (finish_step may be NULL).
 */
int mdl_decode_commit(const int64_t* token, int batch, int64_t* out_ids, int64_t out_ld,
                      int col, const int32_t* counters, int32_t* finish_step, int gen_base,
                      int end_id, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MDLARC_HIP_H */
