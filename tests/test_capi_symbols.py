"""The C-ABI library loads on a machine without a GPU and exports exactly what
include/mdlarc_hip.h declares (no compute calls: those need a GPU)."""

import ctypes

import pytest

from mdlarc_scale_amd import _lib


def _require_lib():
    if not _lib.available():
        pytest.skip("libmdlarc_hip.so not built (python -m mdlarc_scale_amd.build)")


def test_header_declares_every_bound_symbol():
    declared = _lib.header_symbols()
    assert len(declared) == len(set(declared))
    assert sorted(declared) == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    _require_lib()
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _lib.header_symbols():
        assert hasattr(handle, name), f"{name} declared in the header but not exported"


def test_host_only_entry_points():
    """Entry points that do no device work answer without a GPU."""
    _require_lib()
    L = _lib.lib()
    # 200: the q_scale contract of the attention entries carries log2(e), the prefill
    # attention entries take row_holes and out_layout, and the fp32 form's entries exist
    assert L.mdl_version() == 200
    assert L.mdl_error_string(0) == b"ok"
    assert b"head_dim" in L.mdl_error_string(-4)
    # workspace sizing is host arithmetic: one split needs none, several need B*H*splits*66 fp32
    assert L.mdl_attn_decode_workspace_bytes(4, 2, 256, 256) == 0
    assert L.mdl_attn_decode_workspace_bytes(4, 2, 1024, 256) == 4 * 2 * 4 * 66 * 4


def test_argument_errors_are_reported_before_any_launch():
    """Shape / pointer checks return negative codes on the host, without touching a device."""
    _require_lib()
    L = _lib.lib()
    fake = 1 << 20                                  # never dereferenced: rejected first
    assert L.mdl_attn_prefill(fake, fake, fake, 1, 4, 1, 32, 4, None, None, None, 1, fake, 0,
                              None) == -4
    # output layout codes are 0 / 1
    assert L.mdl_attn_prefill(fake, fake, fake, 1, 4, 1, 64, 4, None, None, None, 1, fake, 2,
                              None) == -3
    assert L.mdl_swiglu(None, 16, None, None, None, 1, 8, fake, 0, None) == -1
    assert L.mdl_swiglu(fake, 16, None, None, None, 1, 12, fake, 0, None) == -3
    assert L.mdl_swiglu(fake + 2, 16, None, None, None, 1, 8, fake, 0, None) == -2
    # the tile layout needs whole 32-column blocks of the split row; layout codes are 0 / 1
    assert L.mdl_swiglu(fake, 16, None, None, None, 1, 8, fake, 1, None) == -3
    assert L.mdl_swiglu(fake, 32, None, None, None, 1, 16, fake, 2, None) == -3
    # d_ff above 2^29 would overflow the tiled store's int column arithmetic; a grid above
    # 2^31 - 1 blocks cannot be launched: both refused before any launch
    assert L.mdl_swiglu(fake, 2 ** 31, None, None, None, 1, (1 << 29) + 8, fake, 0, None) == -3
    assert L.mdl_swiglu(fake, 2 ** 29, None, None, None, 2 ** 31 - 1, 1 << 28, fake, 0,
                        None) == -3
    # the bf16 form: d_ff a multiple of 8, at most 65535 blocks of 2048 channels, ld % 8 == 0
    assert L.mdl_swiglu_bf16(fake, 64, None, None, None, 1, 12, fake, None) == -3
    assert L.mdl_swiglu_bf16(fake, 2 ** 30, None, None, None, 1, 65536 * 2048, fake, None) == -3
    assert L.mdl_swiglu_bf16(fake, 36, None, None, None, 1, 16, fake, None) == -2
    assert L.mdl_embed_rmsnorm_bf16(fake, None, fake, None, 14, 0, 1, 1, 36, fake, 1e-5, fake,
                                    fake, None) == -3        # d % 8 != 0
    assert L.mdl_add_rmsnorm(fake, None, None, 1, 8, fake, 1e-5, fake, fake, 1, None) == -3
    assert L.mdl_qkv_rope_cache(fake, 192, None, fake, fake, 1, 4, 1, 64, 32, 32, 8, 10, 10, 12,
                                0.125, fake, fake, fake, 1, 4, 1, None, None) == -5
    # the cache dtype code is MDL_DTYPE_F32 (0) or MDL_DTYPE_BF16 (1)
    assert L.mdl_qkv_rope_cache(fake, 192, None, fake, fake, 1, 4, 1, 64, 32, 32, 8, 10, 10, 12,
                                0.125, fake, fake, fake, 2, 4, 0, None, None) == -7
    assert L.mdl_attn_decode(fake, fake, fake, 1, 1, 64, 1024, None, 0, None, None, None, 5,
                             None, None, 0, 128, fake, 0, None) == -6
    # the no-allocation decode refuses work beyond its 4 MiB static scratch before touching a
    # device: 64 rows x 20 heads x 52 splits x 66 floats needs 17.6 MB
    assert L.mdl_attn_decode_workspace_bytes(64, 20, 6656, 128) > 4 << 20
    assert L.mdl_attn_decode_rope_noalloc(fake, 3840, fake, fake, fake, 32, 32, 8, 10, 10, 12,
                                          0.125, fake, fake, 64, 20, 64, 6656, None, 0, None,
                                          None, None, 5, None, 128, fake, 0, None) == -8
    assert b"scratch" in L.mdl_error_string(-8)
    # K5: k a multiple of 32, n of 4, layout codes 0 / 1, row-major lda >= 2k
    assert L.mdl_gemm_split(fake, 64, 0, fake, 32, 0, fake, 8, 4, 8, 48, 0, None) == -3
    assert L.mdl_gemm_split(fake, 64, 0, fake, 32, 0, fake, 8, 4, 6, 32, 0, None) == -3
    assert L.mdl_gemm_split(fake, 64, 2, fake, 32, 0, fake, 8, 4, 8, 32, 0, None) == -3
    assert L.mdl_gemm_split(fake, 32, 0, fake, 32, 0, fake, 8, 4, 8, 32, 0, None) == -3
    assert L.mdl_gemm_split(fake + 8, 64, 0, fake, 32, 0, fake, 8, 4, 8, 32, 0, None) == -2
    assert L.mdl_gemm_split(None, 0, 1, fake, 0, 1, fake, 8, 4, 8, 32, 0, None) == -1
    assert L.mdl_tile_matrix(fake, 40, 4, 40, fake, None) == -3
    # fused K5 forms: n a multiple of 16 (32 for the residual form), d_ff of 16, x required
    assert L.mdl_gemm_norm(fake, fake, 1e-5, fake, None, fake, 24, None, 4, 24, 32, 0,
                           None) == -3
    assert L.mdl_gemm_norm(None, fake, 1e-5, fake, None, fake, 32, None, 4, 32, 32, 0,
                           None) == -1
    # the low part of an fp32 weight is 16-byte aligned like the weight
    assert L.mdl_gemm_norm(fake, fake, 1e-5, fake, fake + 8, fake, 32, None, 4, 32, 32, 0,
                           None) == -2
    assert L.mdl_gemm_norm_swiglu(fake, fake, 1e-5, fake, None, None, None, fake, 4, 24, 32, 0,
                                  None) == -3
    # d_ff above 2^29 is refused before 2 d_ff can overflow
    assert L.mdl_gemm_norm_swiglu(fake, fake, 1e-5, fake, None, None, None, fake, 4, 1 << 30,
                                  32, 0, None) == -3
    assert L.mdl_gemm_split_swiglu(fake, fake, None, None, None, fake, 4, 1 << 30, 32, 0,
                                   None) == -3
    assert L.mdl_gemm_split_residual(fake, fake, None, fake, None, 4, 48, 32, 0, None) == -3
    assert L.mdl_gemm_split_residual(fake, fake, None, fake + 4, None, 4, 64, 32, 0, None) == -2
    assert L.mdl_gemm_split_residual(fake, fake, fake + 8, fake, None, 4, 64, 32, 0, None) == -2
    # K6 activation parts: 1 (hi) or 2 (hi and lo) only; a row-major hi-only a needs lda >= k
    assert L.mdl_prefill_gemm_split(fake, 64, 0, 3, fake, fake, 32, 4, 32, 32, None) == -3
    assert L.mdl_prefill_gemm_split(fake, 32, 0, 2, fake, fake, 32, 4, 32, 32, None) == -3
    assert L.mdl_prefill_gemm_split(fake, 16, 0, 1, fake, fake, 32, 4, 32, 32, None) == -3
    assert L.mdl_prefill_gemm_split_residual(fake, 64, 1, 0, fake, fake, None, 4, 32, 32,
                                             None) == -3
    assert L.mdl_prefill_gemm_norm_swiglu(fake, fake, 1e-5, 0, fake, None, None, fake, 1, 4, 16,
                                          32, None) == -3
    assert L.mdl_prefill_gemm_norm_swiglu(fake, fake, 1e-5, 1, fake, None, None, fake, 3, 4, 16,
                                          32, None) == -3
    assert L.mdl_gemm_split_tiles() >= 1
    assert 1 <= L.mdl_gemm_split_pick(256, 2304, 768) <= L.mdl_gemm_split_tiles()
    # packed prefill: the per-row starts / offsets and the per-token rows / slots are required
    assert L.mdl_attn_prefill_packed(fake, fake, fake, 1, 4, 1, 64, 4, None, None, None, fake, 1,
                                     fake, 0, None) == -1
    assert L.mdl_attn_prefill_packed(fake, fake, fake, 1, 4, 1, 32, 4, None, None, fake, fake, 1,
                                     fake, 1, None) == -4
    assert L.mdl_qkv_rope_cache_packed(fake, 192, None, fake, fake, 4, None, fake, 1, 1, 64, 32,
                                       32, 8, 10, 10, 12, 0.125, fake, fake, fake, 1, 4,
                                       None) == -1
    assert L.mdl_qkv_rope_cache_packed(fake, 192, None, fake, fake, 4, fake, fake, 1, 1, 32, 32,
                                       32, 8, 10, 10, 12, 0.125, fake, fake, fake, 1, 4,
                                       None) == -4
    # K4f (fp32 attention): head_dim 64 only, q_offset needs kv_start, keys inside the cache,
    # the decode slot inside the cache
    assert L.mdl_attn_prefill_f32(fake, fake, fake, 1, 4, 1, 32, 4, None, None, None, 1, fake, 0,
                                  None) == -4
    assert L.mdl_attn_prefill_f32(fake, fake, fake, 1, 4, 1, 64, 4, None, None, fake, 1, fake, 0,
                                  None) == -1
    assert L.mdl_attn_prefill_f32(fake, fake, fake, 1, 8, 1, 64, 4, None, None, None, 1, fake, 0,
                                  None) == -5
    assert L.mdl_attn_prefill_f32(fake + 4, fake, fake, 1, 4, 1, 64, 4, None, None, None, 1, fake,
                                  0, None) == -2
    assert L.mdl_attn_decode_f32(fake, fake, fake, 1, 1, 64, 4, None, 0, None, 4, None, None, 0,
                                 16, fake, 0, None) == -5
    assert L.mdl_attn_decode_f32(fake, fake, fake, 1, 1, 64, 4, None, 0, None, 0, None, None, 0,
                                 16, fake, 2, None) == -3
    # K4f decode chunks: split_len a positive multiple of 16; several chunks need the workspace
    assert L.mdl_attn_decode_f32(fake, fake, fake, 1, 1, 64, 64, None, 0, None, 0, None, None, 0,
                                 8, fake, 0, None) == -3
    assert L.mdl_attn_decode_f32(fake, fake, fake, 1, 1, 64, 64, None, 0, None, 0, None, None, 0,
                                 16, fake, 0, None) == -6
    assert L.mdl_attn_decode_f32(fake, fake, fake, 1, 1, 64, 64, None, 0, None, 0, None, fake,
                                 1000, 16, fake, 0, None) == -6
    # exact lead attention: q_offset needs kv_start; head_dim 64 only; qkv rows 16-byte aligned
    assert L.mdl_attn_prefill_lead(fake, 192, fake, fake, fake, 32, 32, 8, 10, 10, 12, 0.125, 1, 4,
                                   1, 64, None, None, fake, fake, 0, None) == -1
    assert L.mdl_attn_prefill_lead(fake, 96, fake, fake, fake, 32, 32, 8, 10, 10, 12, 0.125, 1, 4,
                                   1, 32, None, None, None, fake, 0, None) == -4
    assert L.mdl_attn_prefill_lead(fake, 194, fake, fake, fake, 32, 32, 8, 10, 10, 12, 0.125, 1, 4,
                                   1, 64, None, None, None, fake, 0, None) == -2
    assert L.mdl_attn_prefill_lead(fake, 192, fake, fake, fake, 32, 32, 8, 10, 10, 12, 0.125, 1, 4,
                                   1, 64, None, None, None, fake, 3, None) == -3
    with pytest.raises(RuntimeError, match="head_dim"):
        _lib.check(-4, "probe")
