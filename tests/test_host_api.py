"""Host-side API of the drop-in (CPU only): names and signatures the reference's callers use,
state_dict keys, module aliases, input validation that happens before any launch."""

import inspect
import sys
import types

import numpy as np
import pytest
import torch

import mdlarc_scale_amd as M
from mdlarc_scale_amd import compat, inference, transformer
from oracle import data_format as odf


def test_generate_output_signature_matches_reference():
    # src/inference.py:487-499
    params = list(inspect.signature(M.generate_output).parameters)
    assert params == ["model", "input_ids", "positions_3d", "example_ids", "attention_mask",
                      "max_new_tokens", "temperature", "top_k", "stop_on_end", "use_compile",
                      "constraints"]
    sig = inspect.signature(M.generate_output).parameters
    assert sig["max_new_tokens"].default == 900 and sig["temperature"].default == 0.0
    assert sig["stop_on_end"].default is True


def test_forward_signature_and_state_dict_keys():
    # src/transformer.py:562-568 and :523-545
    params = list(inspect.signature(M.TinyTransformer.forward).parameters)
    assert params == ["self", "input_ids", "pos_xyz", "example_ids", "attention_mask",
                      "is_causal"]
    m = M.create_model(d_model=128, n_heads=2, n_layers=2, d_ff=64)
    keys = set(m.state_dict())
    want = {"token_embed.weight", "example_embed.weight", "ln_f.weight", "lm_head.weight"}
    for i in range(2):
        p = f"blocks.{i}."
        want |= {p + "ln1.weight", p + "attn.qkv_proj.weight", p + "attn.out_proj.weight",
                 p + "ln2.weight"}
        want |= {p + f"ffn.fc_{n}.{w}" for n in ("gate", "up", "down") for w in ("weight", "bias")}
    assert keys == want


def test_presets_and_param_count():
    # README.md:74-79 of the reference; tests/test_transformer.py:258-265 (small in 25M..35M)
    small = M.create_small_model()
    assert 25_000_000 < small.num_parameters < 35_000_000
    assert small.num_parameters == 29_342_464
    assert M.create_tiny_model().num_parameters == 3_555_072


def test_autograd_path_runs_on_cpu_and_matches_oracle():
    """With autograd (training / test-time adaptation) forward composes torch ops; on the CPU it
    matches the oracle, and gradients reach example_embed (src/eval.py:144-215)."""
    from oracle import reference_path as rp

    torch.manual_seed(0)
    m = M.create_model(d_model=128, n_heads=2, n_layers=2, d_ff=64, dropout=0.0)
    ids = torch.randint(0, 14, (2, 9))
    pos = torch.randint(0, 30, (2, 9, 3))
    ex = torch.tensor([1, 3])
    mask = torch.ones(2, 9, dtype=torch.bool)
    mask[0, :3] = False
    out = m(ids, pos, ex, mask)
    c = m.config
    om = rp.OracleModel(rp.OracleConfig(c.d_model, c.n_heads, c.n_layers, c.d_ff),
                        m.state_dict())
    ref = om.forward(ids, pos, ex, mask, True)
    assert torch.allclose(out[mask], ref[mask], atol=1e-5)
    out[mask].sum().backward()
    assert m.example_embed.weight.grad is not None
    assert m.example_embed.weight.grad[1].abs().sum() > 0


def test_inference_requires_gpu_tensors_and_fails_loudly():
    m = M.create_tiny_model(dropout=0.0).eval()
    ids = torch.zeros(1, 4, dtype=torch.long)
    pos = torch.zeros(1, 4, 3, dtype=torch.long)
    with torch.no_grad(), pytest.raises(RuntimeError, match="ROCm GPU"):
        m(ids, pos)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        M.generate_output(m, ids, pos, max_new_tokens=4)


def test_generate_output_validation_order():
    """Mask shape is checked and over-long prompts are returned unchanged exactly as the
    reference does (src/inference.py:530-537) -- neither needs a GPU."""
    m = M.create_model(d_model=128, n_heads=2, n_layers=1, d_ff=64, max_seq_len=8)
    ids = torch.zeros(2, 8, dtype=torch.long)
    pos = torch.zeros(2, 8, 3, dtype=torch.long)
    m.eval()
    with pytest.raises(ValueError, match="attention_mask"):
        M.generate_output(m, ids, pos, attention_mask=torch.ones(2, 7, dtype=torch.bool))
    # prompt already fills max_seq_len -> the same tensor comes back, nothing is computed
    assert M.generate_output(m, ids, pos, max_new_tokens=4) is ids
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        M.generate_output(m, ids[:, :5], pos[:, :5], max_new_tokens=4)


def test_ablation_variants_are_rejected():
    with pytest.raises(ValueError, match="unsupported"):
        M.create_model(rope_type="1d")
    with pytest.raises(ValueError, match="unsupported"):
        M.create_model(ffn_type="gelu")


def test_compat_aliases_modules():
    pkg = types.ModuleType("fakeref")
    pkg.__path__ = []
    sys.modules["fakeref"] = pkg
    try:
        compat.install("fakeref")
        assert compat.installed("fakeref")
        from fakeref.inference import generate_output  # noqa: F401
        from fakeref.transformer import TinyTransformer

        assert TinyTransformer is transformer.TinyTransformer
        assert sys.modules["fakeref.inference"] is inference
        compat.install("fakeref")                         # idempotent
    finally:
        for k in [k for k in sys.modules if k == "fakeref" or k.startswith("fakeref.")]:
            del sys.modules[k]


def test_compat_refuses_late_install():
    pkg = types.ModuleType("fakeref2")
    pkg.__path__ = []
    sys.modules["fakeref2"] = pkg
    sys.modules["fakeref2.transformer"] = types.ModuleType("fakeref2.transformer")
    try:
        with pytest.raises(RuntimeError, match="before compat.install"):
            compat.install("fakeref2")
    finally:
        for k in [k for k in sys.modules if k == "fakeref2" or k.startswith("fakeref2.")]:
            del sys.modules[k]


def test_product_data_format_equals_oracle():
    """mdlarc_scale_amd.data (vectorised positions) equals the oracle's scalar restatement."""
    rng = np.random.default_rng(11)
    for _ in range(30):
        toks = []
        for _p in range(rng.integers(1, 4)):
            h, w = rng.integers(1, 33, size=2)
            g = rng.integers(0, 10, size=(h, w)).tolist()
            toks += odf.encode_example(g, g if rng.random() < 0.7 else None)
        assert M.encode_example([[1, 2]], [[3]]) == odf.encode_example([[1, 2]], [[3]])
        assert np.array_equal(M.compute_positions_3d(toks), odf.compute_positions_3d(toks))
        assert M.decode_output_grid(toks) == odf.decode_output_grid(toks)
    sq = [[1, 2, 3], [4, 5, 6]]
    assert [f(sq) for f in M.DIHEDRAL_TRANSFORMS] == [f(sq) for f in odf.DIHEDRAL]
    assert np.array_equal(M.generate_color_permutations(8, 42), odf.color_permutations(8, 42))


def test_workload_specs_meet_their_ranges():
    from mdlarc_scale_amd.workload import SPECS, build_prompts

    for name in ("small_b256", "medium_b128", "large_b64"):
        spec = SPECS[name]
        p = build_prompts(spec)
        lens = [len(t) for t in p]
        assert len(p) == spec.batch
        assert spec.prompt_len[0] <= min(lens) and max(lens) <= spec.prompt_len[1]
        assert max(lens) + 1 < spec.cache_slots
        # positions of every prompt follow the token format
        assert np.array_equal(M.compute_positions_3d(p[0]), odf.compute_positions_3d(p[0]))


def test_reference_private_names_exist_with_their_signatures():
    """The module-level helpers of src/inference.py that code may call or patch
    (:285, :372, :383, :427, :466, :763, :923) exist with the reference's parameters."""
    want = {
        "_apply_logit_constraints": ["logits", "grid_state", "constraints"],
        "_build_sdpa_mask": ["attention_mask", "dtype"],
        "_prefill": ["model", "input_ids", "positions_3d", "example_ids", "cache",
                     "attention_mask"],
        "_decode_step": ["model", "token", "position", "example_ids", "cache",
                         "attention_mask"],
        "_get_decode_fn": ["use_compile"],
        "_predict_augmentations_batched": [
            "model", "task", "test_idx", "device", "example_id", "use_train_examples",
            "num_color_perms", "max_output_tokens", "num_samples", "sample_temperature",
            "sample_top_k", "constrain_decoding", "base_palette", "base_shape",
            "palette_penalty", "shape_penalty", "use_compile", "max_batch_size"],
        "_predict_augmentations_sequential": [
            "model", "task", "test_idx", "device", "example_id", "use_train_examples",
            "num_color_perms", "max_output_tokens", "num_samples", "sample_temperature",
            "sample_top_k", "constrain_decoding", "base_palette", "base_shape",
            "palette_penalty", "shape_penalty", "use_compile"],
    }
    for name, params in want.items():
        assert list(inspect.signature(getattr(inference, name)).parameters) == params, name
    assert inference._get_decode_fn(True) is inference._decode_step
    assert inference._get_decode_fn(False) is inference._decode_step


def test_build_sdpa_mask_closed_form():
    """src/inference.py:372-380: [B, S] bool -> [B, 1, 1, S], 0 where True, -inf where False."""
    m = torch.tensor([[True, False, True], [False, False, True]])
    got = inference._build_sdpa_mask(m, torch.bfloat16)
    assert got.shape == (2, 1, 1, 3) and got.dtype == torch.bfloat16
    want = torch.tensor([[0.0, float("-inf"), 0.0], [float("-inf"), float("-inf"), 0.0]])
    assert torch.equal(got[:, 0, 0].float(), want)
    assert inference._build_sdpa_mask(None, torch.float32) is None


def test_apply_logit_constraints_alias_matches_the_product_rule():
    """_apply_logit_constraints(logits, grid_state, constraints) on [B, 1, V] logits equals
    apply_logit_constraints on the [B, V] rows with the state's x / y, in place."""
    g = torch.Generator().manual_seed(4)
    B = 5
    logits = torch.randn(B, 1, 14, generator=g)
    gx = torch.randint(0, 6, (B,), generator=g)
    gy = torch.randint(0, 6, (B,), generator=g)
    cons = inference.DecodingConstraints(
        palette_mask=torch.rand(B, 10, generator=g) < 0.5,
        target_shape=torch.randint(1, 5, (B, 2), generator=g))
    state = types.SimpleNamespace(x=gx, y=gy)
    want = inference.apply_logit_constraints(logits[:, 0].clone(), gx, gy, cons)
    got = inference._apply_logit_constraints(logits, state, cons)
    assert got is logits and torch.equal(got[:, 0], want)
    assert inference._apply_logit_constraints(logits, state, None) is logits


def test_fp32_form_requires_k5_widths():
    """A model with fp32 parameters runs the fp32 form, whose projections all run on K5: a
    width that is not a multiple of 32 is refused with a clear error before any device work."""
    from mdlarc_scale_amd.engine import PackedWeights, model_form

    m = M.create_model(d_model=128, n_heads=2, n_layers=1, d_ff=200)
    assert model_form(m) == "fp32" and model_form(m.to(torch.bfloat16)) == "bf16"
    with pytest.raises(ValueError, match="multiples of 32"):
        PackedWeights(M.create_model(d_model=128, n_heads=2, n_layers=1, d_ff=200),
                      torch.device("cpu"))
    with pytest.raises(TypeError, match="float32 and bfloat16"):
        model_form(M.create_model(d_model=128, n_heads=2, n_layers=1, d_ff=64).half())
