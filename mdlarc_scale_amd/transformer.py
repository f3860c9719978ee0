"""TinyTransformer with 3D RoPE -- drop-in for src/transformer.py of shyampathak22/mdlARC_scale.

Same class names, constructor arguments, submodule names and ``state_dict`` keys as the reference
(src/transformer.py:15-745), so reference checkpoints load unchanged and ``eval.py`` /
``voting.py`` callers see the same API.

Execution:
* inference (``model.eval()`` with autograd off, e.g. under ``torch.no_grad()``) on a GPU runs the
  HIP kernels of ``libmdlarc_hip.so`` through :mod:`mdlarc_scale_amd.engine`; a missing library
  raises, there is no fallback;
* when autograd is needed (training, the test-time adaptation of example embeddings in the
  reference's eval.py:144-215) or dropout is active, ``forward`` composes the same math from
  differentiable torch ops (the module ``forward`` methods below).  That path exists for gradients;
  it is not the inference hot path and is never chosen as a substitute for a missing library.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class TransformerConfig:
    """Model configuration; field names and defaults of src/transformer.py:15-34."""

    vocab_size: int = 14
    max_seq_len: int = 1863
    d_model: int = 128
    n_heads: int = 4
    d_ff: int = 320
    n_layers: int = 4
    dropout: float = 0.1
    num_examples: int = 1280
    max_x: int = 32
    max_y: int = 32
    max_z: int = 8
    rope_base: float = 10000.0
    norm_eps: float = 1e-5
    rope_type: str = "3d"
    norm_type: str = "rmsnorm"
    ffn_type: str = "swiglu"
    use_example_embedding: bool = True

    def validate(self) -> None:
        if self.d_model % self.n_heads:
            raise ValueError("d_model must be divisible by n_heads")
        unsupported = [(k, v, want) for k, v, want in (
            ("rope_type", self.rope_type.lower(), "3d"),
            ("norm_type", self.norm_type.lower(), "rmsnorm"),
            ("ffn_type", self.ffn_type.lower(), "swiglu")) if v != want]
        if unsupported:
            raise ValueError(
                "mdlarc_scale_amd implements the default architecture (3D RoPE, RMSNorm, SwiGLU); "
                f"unsupported ablation setting(s): {unsupported}")


class RMSNorm(nn.Module):
    """y = x / sqrt(mean(x^2) + eps) * weight (src/transformer.py:37-48)."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        inv = torch.rsqrt(x.square().mean(dim=-1, keepdim=True) + self.eps)
        return x * inv * self.weight


def rope3d_pairs(head_dim: int) -> tuple[int, int, int]:
    """Rotation pairs per axis: n//3 for x and y, the rest for z (src/transformer.py:87-90)."""
    n = head_dim // 2
    return n // 3, n // 3, n - 2 * (n // 3)


def rope3d_axis_table(n_pos: int, pairs: int, base: float) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin [n_pos, pairs] of angle pos / base^(2j / 2pairs) (src/transformer.py:95-126)."""
    width = 2 * pairs
    inv_freq = 1.0 / (base ** (torch.arange(0, width, 2, dtype=torch.float32) / width))
    angle = torch.arange(n_pos, dtype=torch.float32)[:, None] * inv_freq[None, :]
    return angle.cos(), angle.sin()


class RotaryEmbedding3D(nn.Module):
    """3D rotary embedding over (column x, row y, semantic layer z) with interleaved pairs
    (src/transformer.py:61-187).  Buffers cos_x/sin_x/... are non-persistent, as in the
    reference."""

    def __init__(self, head_dim: int, max_x: int = 32, max_y: int = 32, max_z: int = 16,
                 base: float = 10000.0):
        super().__init__()
        self.head_dim, self.base = head_dim, base
        self.max_x, self.max_y, self.max_z = max_x, max_y, max_z
        self.px, self.py, self.pz = rope3d_pairs(head_dim)
        for axis, n_pos, pairs in (("x", max_x, self.px), ("y", max_y, self.py),
                                   ("z", max_z, self.pz)):
            c, s = rope3d_axis_table(n_pos, pairs, base)
            self.register_buffer("cos_" + axis, c, persistent=False)
            self.register_buffer("sin_" + axis, s, persistent=False)

    def device_table(self, device: torch.device) -> torch.Tensor:
        """fp32 [cos_x|sin_x|cos_y|sin_y|cos_z|sin_z], rebuilt in fp32 from the config (the module
        buffers follow the model dtype after ``.to(bfloat16)``; the kernels keep fp32 tables)."""
        parts = []
        for n_pos, pairs in ((self.max_x, self.px), (self.max_y, self.py), (self.max_z, self.pz)):
            c, s = rope3d_axis_table(n_pos, pairs, self.base)
            parts += [c.reshape(-1), s.reshape(-1)]
        return torch.cat(parts).to(device)

    def _angles(self, pos_xyz: torch.Tensor, dtype: torch.dtype):
        ix = pos_xyz[..., 0].clamp(0, self.max_x - 1).long()
        iy = pos_xyz[..., 1].clamp(0, self.max_y - 1).long()
        iz = pos_xyz[..., 2].clamp(0, self.max_z - 1).long()
        cos = torch.cat([self.cos_x[ix], self.cos_y[iy], self.cos_z[iz]], dim=-1)
        sin = torch.cat([self.sin_x[ix], self.sin_y[iy], self.sin_z[iz]], dim=-1)
        return cos.unsqueeze(-2).to(dtype), sin.unsqueeze(-2).to(dtype)

    @staticmethod
    def _rotate(t: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        pairs = t.unflatten(-1, (-1, 2))
        a, b = pairs[..., 0], pairs[..., 1]
        return torch.stack((a * cos - b * sin, b * cos + a * sin), dim=-1).flatten(-2)

    def apply_rotary(self, q: torch.Tensor, k: torch.Tensor,
                     pos_xyz: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Rotate q, k [B, S, H, hd] by positions [B, S, 3] (src/transformer.py:132-187)."""
        cos, sin = self._angles(pos_xyz, q.dtype)
        return self._rotate(q, cos, sin), self._rotate(k, cos, sin)


class MultiHeadSelfAttention(nn.Module):
    """Fused-qkv attention with 3D RoPE (src/transformer.py:245-355)."""

    def __init__(self, config: TransformerConfig):
        super().__init__()
        self.config = config
        self.rope_type = config.rope_type.lower()
        self.n_heads = config.n_heads
        self.head_dim = config.d_model // config.n_heads
        self.scale = self.head_dim ** -0.5
        self.qkv_proj = nn.Linear(config.d_model, 3 * config.d_model, bias=False)
        self.out_proj = nn.Linear(config.d_model, config.d_model, bias=False)
        self.rope = RotaryEmbedding3D(self.head_dim, config.max_x, config.max_y, config.max_z,
                                      config.rope_base)
        self.dropout = nn.Dropout(config.dropout)
        self.k_cache: torch.Tensor | None = None
        self.v_cache: torch.Tensor | None = None

    def forward(self, x: torch.Tensor, pos_xyz: torch.Tensor,
                attention_mask: torch.Tensor | None = None,
                is_causal: bool = True) -> torch.Tensor:
        B, S, D = x.shape
        q, k, v = self.qkv_proj(x).view(B, S, 3, self.n_heads, self.head_dim).unbind(2)
        q, k = self.rope.apply_rotary(q, k, pos_xyz)
        bias = None
        if attention_mask is not None:
            bias = torch.zeros(B, 1, 1, S, dtype=q.dtype, device=x.device)
            bias = bias.masked_fill(~attention_mask.bool()[:, None, None, :], float("-inf"))
        o = F.scaled_dot_product_attention(
            q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), attn_mask=bias,
            dropout_p=self.dropout.p if self.training else 0.0, is_causal=is_causal)
        return self.out_proj(o.transpose(1, 2).reshape(B, S, D))

    def reset_cache(self) -> None:
        self.k_cache = None
        self.v_cache = None


class FeedForward(nn.Module):
    """SwiGLU MLP with biased linears (src/transformer.py:436-451)."""

    def __init__(self, config: TransformerConfig):
        super().__init__()
        self.fc_gate = nn.Linear(config.d_model, config.d_ff)
        self.fc_up = nn.Linear(config.d_model, config.d_ff)
        self.fc_down = nn.Linear(config.d_ff, config.d_model)
        self.dropout = nn.Dropout(config.dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.dropout(self.fc_down(F.silu(self.fc_gate(x)) * self.fc_up(x)))


class TransformerBlock(nn.Module):
    """Pre-norm block: x + attn(ln1 x), then x + ffn(ln2 x) (src/transformer.py:470-497)."""

    def __init__(self, config: TransformerConfig):
        super().__init__()
        self.ln1 = RMSNorm(config.d_model, config.norm_eps)
        self.attn = MultiHeadSelfAttention(config)
        self.ln2 = RMSNorm(config.d_model, config.norm_eps)
        self.ffn = FeedForward(config)
        self.dropout = nn.Dropout(config.dropout)

    def forward(self, x: torch.Tensor, pos_xyz: torch.Tensor,
                attention_mask: torch.Tensor | None = None,
                is_causal: bool = True) -> torch.Tensor:
        x = x + self.dropout(self.attn(self.ln1(x), pos_xyz, attention_mask, is_causal))
        return x + self.dropout(self.ffn(self.ln2(x)))


class TinyTransformer(nn.Module):
    """Decoder-only ARC grid model (src/transformer.py:513-702)."""

    def __init__(self, config: TransformerConfig):
        super().__init__()
        config.validate()
        self.config = config
        self.token_embed = nn.Embedding(config.vocab_size, config.d_model)
        self.example_embed = nn.Embedding(config.num_examples, config.d_model)
        self.blocks = nn.ModuleList([TransformerBlock(config) for _ in range(config.n_layers)])
        self.ln_f = RMSNorm(config.d_model, config.norm_eps)
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)
        self._init_weights()

    def _init_weights(self) -> None:
        """Init distributions of src/transformer.py:547-560: xavier-uniform linear weights, zero
        biases, N(0, 0.02) embeddings, unit norm gains."""
        for mod in self.modules():
            if isinstance(mod, nn.Linear):
                nn.init.xavier_uniform_(mod.weight)
                if mod.bias is not None:
                    nn.init.zeros_(mod.bias)
            elif isinstance(mod, nn.Embedding):
                nn.init.normal_(mod.weight, mean=0.0, std=0.02)
            elif isinstance(mod, RMSNorm):
                nn.init.ones_(mod.weight)

    # -- execution ---------------------------------------------------------------------------
    def _wants_autograd(self) -> bool:
        if self.training:
            return True
        return torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters())

    def forward(self, input_ids: torch.Tensor, pos_xyz: torch.Tensor,
                example_ids: torch.Tensor | None = None,
                attention_mask: torch.Tensor | None = None,
                is_causal: bool = True) -> torch.Tensor:
        """Logits [B, S, vocab] (src/transformer.py:562-599)."""
        if self._wants_autograd():
            return self._forward_autograd(input_ids, pos_xyz, example_ids, attention_mask,
                                          is_causal)
        from .engine import engine_for

        return engine_for(self).forward(input_ids, pos_xyz, example_ids, attention_mask,
                                        is_causal)

    def _forward_autograd(self, input_ids, pos_xyz, example_ids, attention_mask, is_causal):
        x = self.token_embed(input_ids)
        if self.config.use_example_embedding and example_ids is not None:
            x = x + self.example_embed(example_ids).unsqueeze(1)
        for block in self.blocks:
            x = block(x, pos_xyz, attention_mask, is_causal)
        return self.lm_head(self.ln_f(x))

    def reset_cache(self) -> None:
        for block in self.blocks:
            block.attn.reset_cache()

    def refresh_packed_weights(self) -> None:
        """Drop the packed bf16 weight copies used by the HIP path.  Needed only after editing
        weights through ``.data`` (which torch does not version); ``load_state_dict``, ``.to``
        and in-place updates under ``no_grad`` are detected automatically."""
        eng = getattr(self, "_hip_engine", None)
        if eng is not None:
            eng.invalidate()

    @property
    def num_parameters(self) -> int:
        return sum(p.numel() for p in self.parameters() if p.requires_grad)


def create_model(vocab_size: int = 14, d_model: int = 128, n_heads: int = 4, n_layers: int = 4,
                 d_ff: int = 320, dropout: float = 0.1, **kwargs) -> TinyTransformer:
    """Factory with the defaults of src/transformer.py:705-724."""
    cfg = TransformerConfig(vocab_size=vocab_size, d_model=d_model, n_heads=n_heads,
                            n_layers=n_layers, d_ff=d_ff, dropout=dropout, **kwargs)
    return TinyTransformer(cfg)


# model presets of src/transformer.py:728-745
MODEL_SIZES = {
    "tiny": dict(d_model=256, n_heads=4, n_layers=4, d_ff=704),
    "small": dict(d_model=768, n_heads=12, n_layers=4, d_ff=2048),
    "medium": dict(d_model=1024, n_heads=16, n_layers=8, d_ff=2752),
    "large": dict(d_model=1280, n_heads=20, n_layers=12, d_ff=3392),
}


def create_tiny_model(**kwargs) -> TinyTransformer:
    return create_model(**MODEL_SIZES["tiny"], **kwargs)


def create_small_model(**kwargs) -> TinyTransformer:
    return create_model(**MODEL_SIZES["small"], **kwargs)


def create_medium_model(**kwargs) -> TinyTransformer:
    return create_model(**MODEL_SIZES["medium"], **kwargs)


def create_large_model(**kwargs) -> TinyTransformer:
    return create_model(**MODEL_SIZES["large"], **kwargs)


def softmax_scale(head_dim: int) -> float:
    """SDPA's default 1/sqrt(head_dim); 1/8 for head_dim 64, exact in bf16."""
    return 1.0 / math.sqrt(head_dim)


LOG2E = 1.4426950408889634


def attention_q_scale(head_dim: int) -> float:
    """The factor the q producers apply for the attention kernels: the softmax scale times
    log2(e), so the kernels' QK^T products are the exponents of their base-2 softmax."""
    return softmax_scale(head_dim) * LOG2E
