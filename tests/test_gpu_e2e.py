"""End-to-end parity of the HIP inference path (``TinyTransformer.forward`` and
``generate_output`` of mdlarc_scale_amd) against

* the golden vectors written from the reference itself (tests/golden/*.npz: a left-padded ragged
  batch whose ``lengths-1`` rows exercise the reference's right-pad index, per-step logits and
  decode positions, the stop-on-END break), and
* the CPU oracle (oracle/reference_path.py) on the reference's own initialisation for the tiny
  and small presets.

Two forms of the path are covered, chosen as the reference chooses its cache dtype (the model's
parameter dtype, src/inference.py:522): a model with fp32 parameters runs the fp32 form (fp32
weights as hi|lo bf16 pairs, fp32 cache and fp32-MFMA attention) -- BASELINE configuration 0 and
the golden fixtures, written by the fp32 reference; a bf16 model runs the bf16 form (bf16 weights,
q / K / V and cache) -- configurations 2-4, which the bench measures.

Bars: fp32 logits within 2e-2 max-abs of the fp32 CPU reference; greedy
tokens identical on >= 99.5% of positions, every divergence a near-tie (oracle top-2 gap <= 2x the
observed max-abs logit error).  The fp32 form meets the absolute bar on every test, the golden
fixtures included.  The bf16 form meets it on the reference-initialised presets; on the golden
micro model (lm_head scaled x4, logits up to |28|) its bf16 q / K / V put it 1.4e-2 to 3.1e-2
away, so there its logit bar is relative: max-abs error <= 2e-2 * max|logit|.
"""

import numpy as np
import pytest
import torch

from oracle import data_format as odf
from oracle import reference_path as rp
from tests.golden_io import load_e2e

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _model_from_fixture(fx):
    from mdlarc_scale_amd import TinyTransformer, TransformerConfig

    c = fx.cfg
    cfg = TransformerConfig(d_model=c.d_model, n_heads=c.n_heads, n_layers=c.n_layers,
                            d_ff=c.d_ff, num_examples=c.num_examples, max_seq_len=c.max_seq_len,
                            dropout=0.0)
    m = TinyTransformer(cfg)
    m.load_state_dict(fx.weights, strict=True)
    return m.to(DEV).eval()


def _near_tie_ok(ref_logits: torch.Tensor, got: torch.Tensor, ref: torch.Tensor,
                 err: float, min_agree: float | None = 0.995) -> None:
    """Every position where got != ref must be a near-tie of the reference logits, and (against
    the reference: min_agree) they agree on at least 99.5% of the positions."""
    bad = (got != ref).nonzero().tolist()
    for idx in bad:
        lg = ref_logits[tuple(idx)]
        top = lg.topk(2).values
        gap = (top[0] - top[1]).item()
        assert gap <= 2 * err, f"divergence at {idx}: top-2 gap {gap:.4f} > 2 x {err:.4f}"
    if min_agree is not None:
        assert len(bad) <= (1 - min_agree) * got.numel(), \
            f"{len(bad)} of {got.numel()} argmaxes differ"


FORMS = ["bf16", "fp32"]


def _preset_model(preset, form, seed=0, max_seq_len=4096):
    """A preset under the reference's initialisation (torch.manual_seed(seed)) in one form:
    "fp32" keeps its fp32 parameters as they are (the reference's configuration 0), "bf16"
    converts it with .to(bfloat16) (configurations 2-4).  Returns the GPU model and the fp32
    state of exactly those weights for the oracle."""
    from mdlarc_scale_amd import create_model
    from mdlarc_scale_amd.transformer import MODEL_SIZES

    torch.manual_seed(seed)
    m = create_model(**MODEL_SIZES[preset], dropout=0.0, max_seq_len=max_seq_len)
    if form == "bf16":
        m = m.to(torch.bfloat16)
    state = {k: v.float().clone() for k, v in m.state_dict().items()}
    return m.to(DEV).eval(), state


def _oracle_of(m, state):
    c = m.config
    return rp.OracleModel(rp.OracleConfig(c.d_model, c.n_heads, c.n_layers, c.d_ff,
                                          c.num_examples, c.max_seq_len), state)


def _fwd(m, ids, pos, ex, mask, causal=True):
    """The HIP forward's fp32 logits on the CPU (a bf16 model's own forward returns its logits
    in bf16, as the reference's does; parity is judged on the fp32 values)."""
    from mdlarc_scale_amd.engine import engine_for

    with torch.no_grad():
        return engine_for(m).forward_f32(
            ids.to(DEV), pos.to(DEV), None if ex is None else ex.to(DEV),
            None if mask is None else mask.to(DEV), causal).float().cpu()


@pytest.mark.parametrize("name", ["e2e_micro", "e2e_micro_stop"])
def test_forward_matches_golden(name):
    fx = load_e2e(name)
    m = _model_from_fixture(fx)
    with torch.no_grad():
        got = m(fx.ids.to(DEV), fx.pos.to(DEV), fx.ex_ids.to(DEV), fx.mask.to(DEV), True)
    got = got.float().cpu()
    err = (got - fx.fwd_logits).abs()
    valid = fx.mask                                    # pad query rows are not compared
    e = err[valid].max().item()
    print(f"{name}: forward max-abs {e:.4e} (max |logit| {fx.fwd_logits.abs().max():.2f})")
    assert e <= 2e-2                                   # the fixture model is fp32: fp32 form
    assert torch.isfinite(got).all()                   # fully-masked pad rows stay finite


def _golden_teacher_forced(m, fx):
    """The GPU forward over the golden token stream: logits at every decoded position
    ([B, g, V]; the first from row lengths-1, the reference's index on left-padded batches) and
    their max-abs error against the golden per-step logits."""
    S = fx.ids.shape[1]
    B = fx.ids.shape[0]
    g = fx.step_logits.shape[1]
    toks = fx.gen[:, :S + g - 1]
    pos = torch.cat([fx.pos, fx.step_pos], 1)
    mask = torch.cat([fx.mask, torch.ones(B, g - 1, dtype=torch.bool)], 1)
    with torch.no_grad():
        lg = m(toks.to(DEV), pos.to(DEV), fx.ex_ids.to(DEV), mask.to(DEV), True).float().cpu()
    n = fx.mask.sum(1)
    first = lg[torch.arange(B), n - 1]
    steps = torch.cat([first[:, None], lg[:, S:S + g - 1]], 1)
    return steps, (steps - fx.step_logits).abs().max().item()


@pytest.mark.parametrize("name", ["e2e_micro", "e2e_micro_stop"])
def test_generate_matches_golden(name):
    """Free-running greedy tokens equal the reference's, or each row's first divergence is a
    near-tie of the golden logits: top-2 gap <= 2x the teacher-forced max-abs logit error."""
    from mdlarc_scale_amd import generate_output

    fx = load_e2e(name)
    m = _model_from_fixture(fx)
    with torch.no_grad():
        out = generate_output(m, fx.ids.to(DEV), fx.pos.to(DEV), fx.ex_ids.to(DEV),
                              attention_mask=fx.mask.to(DEV), max_new_tokens=fx.max_new)
    out = out.cpu()
    S = fx.ids.shape[1]
    assert torch.equal(out[:, :S], fx.ids)
    n = min(out.shape[1], fx.gen.shape[1])
    got, ref = out[:, S:n], fx.gen[:, S:n]
    agree = (got == ref).float().mean().item()
    print(f"{name}: greedy agreement {agree:.4f} over {got.numel()} tokens")
    if out.shape[1] == fx.gen.shape[1] and torch.equal(out, fx.gen):
        return
    # divergence: the first differing token of each row must be a near-tie in the golden logits
    _, err = _golden_teacher_forced(m, fx)
    for b in range(out.shape[0]):
        diff = (got[b] != ref[b]).nonzero()
        if len(diff):
            t = int(diff[0])
            top = fx.step_logits[b, t].topk(2).values
            gap = (top[0] - top[1]).item()
            assert gap <= 2 * err, f"row {b} step {t}: top-2 gap {gap:.4f} > 2 x {err:.4f}"


def test_generate_teacher_forced_logits_vs_golden():
    """Feed the golden tokens through the GPU forward (teacher forcing): the logits at every
    decoded position match the golden per-step logits, and the argmax agrees except at ties."""
    fx = load_e2e("e2e_micro")
    m = _model_from_fixture(fx)
    # the reference reads its first token at index lengths-1 (right-pad index on a left-padded
    # batch); later steps read the last column
    steps, err = _golden_teacher_forced(m, fx)
    scale = fx.step_logits.abs().max().item()
    agree = (steps.argmax(-1) == fx.step_logits.argmax(-1)).float().mean().item()
    print(f"teacher-forced max-abs {err:.4e} (max |logit| {scale:.2f}), argmax agreement "
          f"{agree:.4f}")
    assert err <= 2e-2
    _near_tie_ok(fx.step_logits, steps.argmax(-1), fx.step_logits.argmax(-1), err)


def test_generate_single_row_defaults():
    """No mask and no example ids: example id defaults to 0 (reference golden)."""
    from mdlarc_scale_amd import generate_output

    fx = load_e2e("e2e_micro")
    m = _model_from_fixture(fx)
    p = fx.single_prompt
    pos = torch.from_numpy(odf.compute_positions_3d(p.tolist()))[None]
    with torch.no_grad():
        out = generate_output(m, p[None].to(DEV), pos.to(DEV), max_new_tokens=12).cpu()
    assert out.shape == fx.single_gen.shape
    S = p.numel()
    # the oracle reproduces the reference's tokens here; its logits decide near-ties
    tr = rp.generate_output(_oracle_of(m, {k: v.clone() for k, v in fx.weights.items()}),
                            p[None], pos, torch.zeros(1, dtype=torch.long), None, 12)
    assert torch.equal(tr.tokens, fx.single_gen)
    g = len(tr.step_logits)
    toks = tr.tokens[:, :S + g - 1]
    tpos = torch.cat([pos, torch.stack(tr.step_positions, 1)], 1)
    steps = _fwd(m, toks, tpos, torch.zeros(1, dtype=torch.long), None)[:, S - 1:S + g - 1]
    ref = torch.stack(tr.step_logits, 1)
    err = (steps - ref).abs().max().item()
    agree = (out[:, S:] == fx.single_gen[:, S:]).float().mean().item()
    print(f"single row: teacher-forced max-abs {err:.3e}, free-running agreement {agree:.4f}")
    assert err <= 2e-2
    _near_tie_ok(ref, steps.argmax(-1), ref.argmax(-1), err)
    assert agree >= 0.995 or _first_divergence_is_tie(out, tr, S, err)


def _random_prompts(rng, B, n_pairs, lo, hi):
    prompts = []
    for _ in range(B):
        toks = []
        for _p in range(n_pairs):
            h, w = rng.integers(lo, hi + 1, size=2)
            gi = rng.integers(1, 10, size=(h, w))
            gi[rng.random((h, w)) < 0.5] = 0
            h2, w2 = rng.integers(lo, hi + 1, size=2)
            go = rng.integers(1, 10, size=(h2, w2))
            go[rng.random((h2, w2)) < 0.5] = 0
            toks += odf.encode_example(gi.tolist(), go.tolist())
        h, w = rng.integers(lo, hi + 1, size=2)
        gt = rng.integers(0, 10, size=(h, w))
        toks += odf.encode_example(gt.tolist(), None)
        prompts.append(toks)
    return prompts


def _left_pad(prompts):
    S = max(len(p) for p in prompts)
    B = len(prompts)
    ids = np.full((B, S), 13, dtype=np.int64)
    pos = np.zeros((B, S, 3), dtype=np.int64)
    mask = np.zeros((B, S), dtype=bool)
    for b, p in enumerate(prompts):
        ids[b, S - len(p):] = p
        pos[b, S - len(p):] = odf.compute_positions_3d(p)
        mask[b, S - len(p):] = True
    return torch.from_numpy(ids), torch.from_numpy(pos), torch.from_numpy(mask)


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("preset", ["tiny", "small"])
def test_reference_init_generate_vs_oracle(preset, form):
    """Reference initialisation (src/transformer.py:547-560) under torch.manual_seed(0), the
    model's weights shared with the fp32 oracle: logits within 2e-2 max-abs at every decoded
    step (teacher-forced through the oracle's tokens) and >= 99.5% greedy agreement."""
    m, state = _preset_model(preset, form)
    rng = np.random.default_rng(20261201)
    ids, pos, mask = _left_pad(_random_prompts(rng, 4, 3, 1, 8))
    ex = torch.tensor([0, 5, 17, 1279])
    _compare_with_oracle(m, state, ids, pos, ex, mask, 48, f"{preset} {form}")


def _compare_with_oracle(m, state, ids, pos, ex, mask, max_new, label):
    """GPU generate_output against the fp32 oracle's: teacher-forced logits (the GPU forward
    over the oracle's token stream) within 2e-2 max-abs at every decoded step with every
    argmax difference a near-tie, and >= 99.5% free-running greedy agreement (or a near-tie at
    each row's first divergence)."""
    from mdlarc_scale_amd import generate_output

    B = ids.shape[0]
    om = _oracle_of(m, state)
    tr = rp.generate_output(om, ids, pos, ex, mask, max_new)
    with torch.no_grad():
        out = generate_output(m, ids.to(DEV), pos.to(DEV), ex.to(DEV), attention_mask=mask.to(DEV),
                              max_new_tokens=max_new).cpu()
    S = ids.shape[1]
    n = min(out.shape[1], tr.tokens.shape[1])
    agree = (out[:, S:n] == tr.tokens[:, S:n]).float().mean().item()
    # teacher-forced logits: GPU forward over the oracle's token stream
    g = len(tr.step_logits)
    toks = tr.tokens[:, :S + g - 1]
    tpos = torch.cat([pos, torch.stack(tr.step_positions, 1)], 1) if g > 1 else pos
    tmask = torch.cat([mask, torch.ones(B, g - 1, dtype=torch.bool)], 1)
    lg = _fwd(m, toks, tpos, ex, tmask)
    first = lg[torch.arange(B), mask.sum(1) - 1]
    steps = torch.cat([first[:, None], lg[:, S:S + g - 1]], 1)
    ref = torch.stack(tr.step_logits, 1)
    err = (steps - ref).abs().max().item()
    print(f"{label}: teacher-forced logits max-abs {err:.3e}, free-running agreement {agree:.4f}")
    assert err <= 2e-2
    _near_tie_ok(ref, steps.argmax(-1), ref.argmax(-1), err)
    assert agree >= 0.995 or _first_divergence_is_tie(out, tr, S, err)


@pytest.mark.parametrize("form", FORMS)
def test_generate_with_mask_holes_vs_oracle(form):
    """Prompt masks with holes inside the valid run (the reference accepts any boolean mask,
    src/inference.py:530-531, :557-558): the packed prefill keeps the holes as masked keys, decode
    reads the mask per slot for rows with holes, and lengths-1 counts valid positions only, so it
    moves left of the last token.  One row starts with a hole (its first valid position moves
    right), one has none.  Tiny reference-initialised model against the fp32 oracle."""
    m, state = _preset_model("tiny", form, seed=1)
    rng = np.random.default_rng(77)
    ids, pos, mask = _left_pad(_random_prompts(rng, 5, 3, 1, 8))
    for b in range(1, 5):
        valid = mask[b].nonzero().flatten()
        k = min(7, len(valid) - 2)
        if k > 0:
            mask[b, torch.from_numpy(rng.choice(valid[1:-1].numpy(), size=k, replace=False))] = False
    first = mask[2].nonzero().flatten()[0]
    mask[2, first:first + 3] = False                 # row 2 starts with holes
    assert all(int(mask[b].sum()) > 0 for b in range(5))
    ex = torch.tensor([3, 0, 9, 100, 1279])
    _compare_with_oracle(m, state, ids, pos, ex, mask, 40, f"holes {form}")


def _first_divergence_is_tie(out, tr, S, err):
    ref = torch.stack(tr.step_logits, 1)
    for b in range(out.shape[0]):
        n = min(out.shape[1], tr.tokens.shape[1])
        d = (out[b, S:n] != tr.tokens[b, S:n]).nonzero()
        if len(d):
            t = int(d[0])
            top = ref[b, t].topk(2).values
            if (top[0] - top[1]).item() > 2 * err:
                return False
    return True


def test_generate_properties_of_the_reference_suite():
    """The properties the reference's own tests pin for generate_output and predict_grid
    (tests/test_inference.py): output length within [S, S + max_new] (:55-80); greedy
    determinism across calls, also after an unrelated call of another shape in between (:82-98,
    :301-363); a right-padded B=2 batch padded with token 0 and no mask (:100-123), whose prompt
    comes back unchanged; predict_grid returns a grid (list of lists) or None (:155-214)."""
    from mdlarc_scale_amd import create_tiny_model, generate_output, predict_grid

    torch.manual_seed(0)
    m = create_tiny_model(dropout=0.0).to(DEV).eval()
    rng = np.random.default_rng(5)
    ids, pos, mask = _left_pad(_random_prompts(rng, 3, 2, 1, 5))
    ids, pos, mask = ids.to(DEV), pos.to(DEV), mask.to(DEV)
    S = ids.shape[1]
    with torch.no_grad():
        a = generate_output(m, ids, pos, None, mask, max_new_tokens=25)
        generate_output(m, ids[:1, -5:], pos[:1, -5:], max_new_tokens=7)
        b = generate_output(m, ids, pos, None, mask, max_new_tokens=25)
    assert S < a.shape[1] <= S + 25
    assert torch.equal(a, b)
    assert torch.equal(a[:, :S], ids)
    p1 = odf.encode_example([[1, 2], [3, 4]], None)
    p2 = odf.encode_example([[5]], None)
    L = max(len(p1), len(p2))
    ids2 = torch.zeros(2, L, dtype=torch.long)
    pos2 = torch.zeros(2, L, 3, dtype=torch.long)
    for r, p in enumerate((p1, p2)):
        ids2[r, :len(p)] = torch.tensor(p)
        pos2[r, :len(p)] = torch.from_numpy(odf.compute_positions_3d(p))
    with torch.no_grad():
        out2 = generate_output(m, ids2.to(DEV), pos2.to(DEV), max_new_tokens=10).cpu()
    assert out2.shape[0] == 2 and L < out2.shape[1] <= L + 10
    assert torch.equal(out2[:, :L], ids2)
    assert int(out2.min()) >= 0 and int(out2.max()) < 14
    g = predict_grid(m, [[[1, 2], [3, 4]]], [[[4, 3], [2, 1]]], [[5, 6], [7, 8]], DEV,
                     max_output_tokens=20)
    assert g is None or (isinstance(g, list) and all(isinstance(row, list) for row in g))


@pytest.mark.parametrize("form", FORMS)
def test_sampling_paths(form):
    """The sampling branch (src/inference.py:575-583) runs the host-launched decode step: with
    top_k = 1 it must return exactly the greedy tokens of the captured path; with a temperature
    and no top-k it draws from torch's generator, so the same seed gives the same tokens, all
    inside the vocabulary."""
    from mdlarc_scale_amd import generate_output

    m, _ = _preset_model("small", form, seed=6, max_seq_len=1024)
    rng = np.random.default_rng(6)
    ids, pos, mask = _left_pad(_random_prompts(rng, 5, 2, 1, 6))
    ids, pos, mask = ids.to(DEV), pos.to(DEV), mask.to(DEV)
    ex = torch.arange(5, device=DEV)
    with torch.no_grad():
        greedy = generate_output(m, ids, pos, ex, mask, max_new_tokens=30, stop_on_end=False)
        top1 = generate_output(m, ids, pos, ex, mask, max_new_tokens=30, temperature=0.8,
                               top_k=1, stop_on_end=False)
        runs = []
        for _ in range(2):
            torch.manual_seed(123)
            runs.append(generate_output(m, ids, pos, ex, mask, max_new_tokens=30,
                                        temperature=1.3, stop_on_end=False))
    assert torch.equal(top1, greedy)
    assert torch.equal(runs[0], runs[1])
    S = ids.shape[1]
    assert runs[0].shape == greedy.shape
    assert int(runs[0][:, S:].min()) >= 0 and int(runs[0][:, S:].max()) < 14


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("preset", ["tiny", "small", "medium", "large"])
def test_forward_presets_vs_oracle(preset, form):
    """model.forward at every position of short unpadded prompts, all four presets under
    reference init with weights shared with the fp32 oracle: logits within 2e-2.  In the bf16
    form the first positions carry the largest error (causal attention there returns a single
    bf16 V row, with nothing to average its rounding), so this pins the worst positions the path
    has.  A bf16 model's own forward returns bf16 logits, as the reference's does."""
    m, state = _preset_model(preset, form, max_seq_len=1024)
    rng = np.random.default_rng(100)
    prompts = _random_prompts(rng, 3, 2, 2, 6)
    L = min(len(p) for p in prompts)
    ids = torch.tensor([p[-L:] for p in prompts], dtype=torch.long)
    pos = torch.stack([torch.from_numpy(odf.compute_positions_3d(p[-L:])) for p in prompts])
    ex = torch.tensor([0, 1, 5])
    ref = _oracle_of(m, state).forward(ids, pos, ex, None, True)
    got = _fwd(m, ids, pos, ex, None)
    err = (got - ref).abs()
    worst = int(err.amax(-1).amax(0).argmax())
    print(f"{preset} {form} forward, {L} positions: logits max-abs {err.max().item():.3e} "
          f"(position {worst}), mean {err.mean().item():.2e}")
    assert err.max().item() <= 2e-2
    with torch.no_grad():
        own = m(ids.to(DEV), pos.to(DEV), ex.to(DEV), None, True)
    assert own.dtype == next(m.parameters()).dtype
    assert torch.equal(own.float().cpu(), got.to(own.dtype).float())


@pytest.mark.parametrize("form", FORMS)
def test_forward_non_causal_vs_oracle(form):
    """TinyTransformer.forward with is_causal=False (src/transformer.py:562-599 passes it to SDPA):
    every query sees every valid key of its row, padding queries included.  Tiny
    reference-initialised model, weights shared with the fp32 oracle: logits within 2e-2."""
    m, state = _preset_model("tiny", form, seed=2, max_seq_len=1024)
    rng = np.random.default_rng(8)
    ids, pos, mask = _left_pad(_random_prompts(rng, 4, 2, 1, 6))
    ex = torch.tensor([1, 2, 3, 4])
    ref = _oracle_of(m, state).forward(ids, pos, ex, mask, is_causal=False)
    got = _fwd(m, ids, pos, ex, mask, causal=False)
    err = (got - ref).abs().max().item()
    print(f"non-causal forward ({form}): logits max-abs {err:.3e}")
    assert err <= 2e-2


def test_autograd_forward_on_gpu():
    """With autograd on -- test-time adaptation of the example embedding, src/eval.py:144-215 --
    forward composes torch ops on the GPU instead of the kernels: its logits agree with the
    kernel path to the parity bar, and the gradient reaches exactly the example-embedding rows
    the batch uses."""
    from mdlarc_scale_amd import create_tiny_model

    torch.manual_seed(3)
    m = create_tiny_model(dropout=0.0)               # fp32: the kernels run the fp32 form
    state = {k: v.clone() for k, v in m.state_dict().items()}
    m = m.to(DEV).eval()
    rng = np.random.default_rng(3)
    prompts = _random_prompts(rng, 3, 2, 2, 5)
    L = min(len(p) for p in prompts)
    ids = torch.tensor([p[-L:] for p in prompts], dtype=torch.long)
    pos = torch.stack([torch.from_numpy(odf.compute_positions_3d(p[-L:])) for p in prompts])
    ids, pos = ids.to(DEV), pos.to(DEV)
    ex = torch.tensor([4, 9, 4], device=DEV)
    with torch.no_grad():
        kern = m(ids, pos, ex, None, True).float()
    m.zero_grad(set_to_none=True)
    out = m(ids, pos, ex, None, True)
    assert out.requires_grad
    c = m.config
    om = rp.OracleModel(rp.OracleConfig(c.d_model, c.n_heads, c.n_layers, c.d_ff,
                                        c.num_examples, c.max_seq_len), state)
    ref = om.forward(ids.cpu(), pos.cpu(), ex.cpu(), None, True)
    e_kern = (kern.cpu() - ref).abs().max().item()
    e_grad = (out.detach().float().cpu() - ref).abs().max().item()
    print(f"logits max-abs vs the fp32 oracle: kernel path {e_kern:.3e}, autograd path "
          f"{e_grad:.3e}")
    assert e_kern <= 2e-2 and e_grad <= 2e-2
    out.float().logsumexp(-1).mean().backward()
    g = m.example_embed.weight.grad
    used = torch.zeros(g.shape[0], dtype=torch.bool, device=DEV)
    used[ex] = True
    assert bool(torch.isfinite(g).all())
    assert bool((g[used].abs().sum(1) > 0).all()) and bool((g[~used] == 0).all())


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("stop_on_end", [True, False])
def test_graph_replay_matches_eager_launches(stop_on_end, form):
    """Greedy decode replayed from one captured HIP graph returns exactly the tokens of the
    eagerly launched step, over many replays with host syncs (the stop check) between them."""
    from mdlarc_scale_amd import generate_output
    from mdlarc_scale_amd import inference as inf

    m, _ = _preset_model("small", form, seed=3, max_seq_len=1024)
    rng = np.random.default_rng(5)
    ids, pos, mask = _left_pad(_random_prompts(rng, 8, 2, 1, 6))
    ex = torch.arange(8)
    outs = []
    for use_graphs in (False, True):
        inf.USE_GRAPHS = use_graphs
        try:
            with torch.no_grad():
                outs.append(generate_output(m, ids.to(DEV), pos.to(DEV), ex.to(DEV),
                                            attention_mask=mask.to(DEV), max_new_tokens=60,
                                            stop_on_end=stop_on_end).cpu())
        finally:
            inf.USE_GRAPHS = True
    assert outs[0].shape == outs[1].shape
    assert torch.equal(outs[0], outs[1])


def test_graph_capture_keeps_allocator_cache(monkeypatch):
    """Capturing the greedy step returns no cached memory to the driver: releasing it slows every
    later HBM-bound kernel of the process, so the capture must not empty torch's cache (the
    ``torch.cuda.graph`` context does) and the reserved pool may not shrink across a generate."""
    from mdlarc_scale_amd import generate_output
    from mdlarc_scale_amd import inference as inf

    m, _ = _preset_model("small", "bf16", seed=3, max_seq_len=1024)
    rng = np.random.default_rng(7)
    ids, pos, mask = _left_pad(_random_prompts(rng, 8, 2, 1, 6))
    calls = []
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: calls.append(1))
    assert inf.USE_GRAPHS
    with torch.no_grad():
        generate_output(m, ids.to(DEV), pos.to(DEV), torch.arange(8).to(DEV),
                        attention_mask=mask.to(DEV), max_new_tokens=20, stop_on_end=False)
        torch.cuda.synchronize()
        reserved = torch.cuda.memory_reserved()
        generate_output(m, ids.to(DEV), pos.to(DEV), torch.arange(8).to(DEV),
                        attention_mask=mask.to(DEV), max_new_tokens=20, stop_on_end=False)
        torch.cuda.synchronize()
    assert not calls
    assert torch.cuda.memory_reserved() >= reserved


def test_predict_with_augmentations_pipeline():
    """The batched augmentation caller runs on the HIP path and returns 8 x perms results with
    the reference's tuple structure (tests/test_inference.py:225-293 of the reference)."""
    from mdlarc_scale_amd import create_tiny_model, predict_with_augmentations

    torch.manual_seed(0)
    m = create_tiny_model(dropout=0.0).to(DEV).eval()
    task = {"train": [{"input": [[1, 2], [3, 4]], "output": [[4, 3], [2, 1]]},
                      {"input": [[5, 0], [0, 5]], "output": [[0, 5], [5, 0]]}],
            "test": [{"input": [[6, 7], [8, 9]]}]}
    preds = predict_with_augmentations(m, task, 0, DEV, num_color_perms=2, max_output_tokens=20)
    assert len(preds) == 16
    assert [p[1] for p in preds[::2]] == list(range(8))
    assert preds[0][2] is None and preds[1][2] is not None


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("r", range(7))
def test_augmentations_vs_reference_golden(r, form, monkeypatch):
    """predict_with_augmentations (src/inference.py:697-1003) against what the reference itself
    produced (tests/golden/augment_micro.npz) on the micro model with bf16-rounded weights (in an
    fp32 model, as the reference ran it): the batched chunk loop at chunk sizes 16 and 5 and the
    sequential loop, constraints on and off, a model that ends rows at many different steps and
    one that runs into the max_seq_len budgets.  The product runs every variant in ONE
    generation (each row keeping its chunk's lengths-1 row, budget and stop step); the test grid
    1x5 becomes 5x1 under half the transforms, so chunks differ in width and budget.  "fp32" runs
    the fixture's fp32 model (the fp32 form); "bf16" the same weights as a bf16 model (exact: they
    are bf16 values), whose bf16 q / K / V put it within the relative bar only.

    * Teacher-forced: the product's decode path over the fused batch (row_shift as the product
      sets it) fed the reference's tokens; its logits lie within 2e-2 (fp32 form; bf16 form:
      2e-2 * max|logit|) of the oracle's at every step the reference decoded (the oracle
      reproduces the fixture's token streams exactly, tests/test_oracle.py), and the argmax of
      its constrained logits equals the reference's token on >= 99.5% of the steps, every
      difference a near-tie of the reference's constrained logits.  The bf16 form keeps the
      near-tie rule but not the 99.5%: on this model, whose logits are 3-5x larger than the
      presets', its bf16 q / K / V flip 0.1-2.3% of the argmaxes between near-tied tokens (the
      fp32 form, the fixture's own, flips none).
    * Free-running: per variant, the dihedral / permutation labels equal the reference's; the
      generated tokens equal the reference's up to a first divergence that must be a near-tie of
      the reference's constrained logits (top-2 gap <= 2x the teacher-forced error); the raw
      stream each prediction is decoded from (decode_output_grid replaced by the identity)
      equals the reference's in every chunk without such a divergence."""
    from mdlarc_scale_amd import inference as inf
    from oracle import augment as oa
    from tests.golden_io import load_augment

    fx = load_augment()
    run = fx.runs[r]
    m, om = _micro_model(run.stop_model, form)
    kw = dict(example_id=fx.example_id, num_color_perms=fx.num_color_perms,
              max_output_tokens=fx.max_new, constrain_decoding=run.constrain,
              batched=run.batched, max_batch_size=run.chunk)
    otr = oa.predict_with_augmentations(om, fx.task, 0, decode=lambda toks: tuple(toks), **kw)
    assert otr.generated == run.gen                      # the oracle is the reference here
    n, chunk = len(run.gen), run.chunk

    # teacher-forced logits of the fused batch
    ids, pos, mask = _left_pad(otr.prompts)
    S = ids.shape[1]
    shift = torch.tensor([S - w for w in otr.widths], dtype=torch.int32)
    steps = max(len(gn) for gn in run.gen)
    toks = torch.full((n, S + steps), 13, dtype=torch.long)
    toks[:, :S] = ids
    for i, gn in enumerate(run.gen):
        toks[i, S:S + len(gn)] = torch.tensor(gn)
    ex = torch.full((n,), fx.example_id, dtype=torch.long)
    raw, _, _ = _teacher_forced_decode(m, ids, pos, ex, mask, toks, steps, S + steps,
                                       row_shift=shift)
    err, scale = 0.0, 0.0
    for i, gn in enumerate(run.gen):
        k = len(gn)
        err = max(err, (raw[i, :k] - otr.raw_logits[i]).abs().max().item())
        scale = max(scale, otr.raw_logits[i].abs().max().item())
    assert err <= (2e-2 if form == "fp32" else 2e-2 * scale)
    # teacher-forced argmax: the grid state is the reference's at every step, so the constraint
    # penalties are the reference's -- the product's constrained logits are its raw logits plus
    # the reference's (constrained - raw) difference (-inf where the reference disallows)
    tf_total, tf_bad = 0, 0
    for i, gn in enumerate(run.gen):
        k = len(gn)
        ref_c, ref_r = otr.step_logits[i], otr.raw_logits[i]
        mine = torch.where(torch.isinf(ref_c), ref_c, raw[i, :k] + (ref_c - ref_r))
        pick = mine.argmax(-1)
        tf_total += k
        for t in (pick != torch.tensor(gn)).nonzero().flatten().tolist():
            tf_bad += 1
            gap = float(run.gaps[i][t])
            assert gap <= 2 * err, f"variant {i} step {t}: teacher-forced argmax differs, " \
                                   f"top-2 gap {gap:.4f} > 2 x {err:.4f}"
    if form == "fp32":      # the form the fixture was written in
        assert tf_bad <= 0.005 * tf_total, \
            f"{tf_bad} of {tf_total} teacher-forced argmaxes differ"

    # free-running product call
    seen = {}
    orig = inf._generate

    def capture(*a, **k):
        res = orig(*a, **k)
        seen["out"], seen["S"] = res[0].cpu(), a[1].shape[1]
        return res

    monkeypatch.setattr(inf, "_generate", capture)
    monkeypatch.setattr(inf, "decode_output_grid", lambda toks: tuple(toks))
    preds = inf.predict_with_augmentations(m, fx.task, 0, DEV, **kw)
    assert [(p[1], p[2]) for p in preds] == run.aug
    gen = seen["out"][:, seen["S"]:]
    diverged, total, same = set(), 0, 0
    for i, ref in enumerate(run.gen):
        mine = gen[i, :len(ref)].tolist()
        k = next((j for j, (a, b) in enumerate(zip(mine, ref)) if a != b), None)
        lim = len(mine) if k is None else k
        total += len(ref)
        same += sum(a == b for a, b in zip(mine[:lim], ref[:lim]))
        if k is not None:
            gap = float(run.gaps[i][k])
            assert gap <= 2 * err, f"variant {i} step {k}: top-2 gap {gap:.4f} > 2 x {err:.4f}"
            diverged.add(i // chunk)
        else:
            assert len(mine) == len(ref), f"variant {i}: {len(mine)} of {len(ref)} tokens"
    for i, p in enumerate(preds):
        if i // chunk not in diverged:
            assert p[0] == run.streams[i], f"variant {i}"
    # the product's own chunk-by-chunk loop (sampling takes it) returns the same
    monkeypatch.setattr(inf, "_generate", orig)
    loop = inf.predict_with_augmentations(m, fx.task, 0, DEV, fuse_chunks=False, **kw)
    if not diverged:
        assert loop == preds
    print(f"augment run {r} ({form}): teacher-forced max-abs {err:.3e} (max |logit| "
          f"{scale:.1f}), teacher-forced argmax {tf_total - tf_bad}/{tf_total}, free-running "
          f"{same}/{total} tokens equal, {len(diverged)} chunk(s) with a near-tie divergence")


def _teacher_forced_decode(m, ids, pos, ex, mask, tokens, steps, total, row_shift=None,
                           positions=None):
    """Per-step logits (before any constraint) of the product's decode path -- prefill, then
    grid step, the decode layers (fused K2 + decode attention over the static cache, K5
    projections) and the head, launched eagerly -- fed ``tokens`` [B, S + steps - 1] (the
    prompt, then one token per step per row) instead of its own argmax: [B, steps, V] fp32,
    plus the grid state (x, y) after each step's input token, [B, steps] each.  With
    ``positions`` ([B, steps - 1, 3]) the decode positions are checked equal to them."""
    from mdlarc_scale_amd import kernels as Kn
    from mdlarc_scale_amd.engine import engine_for
    from mdlarc_scale_amd.inference import Generator

    S = ids.shape[1]
    eng = engine_for(m)
    gen = Generator(m)
    got, gxs, gys = [], [], []
    with torch.no_grad():
        W = eng.packed(torch.device(DEV))
        idsd, posd = ids.to(DEV), pos.to(DEV)
        st = gen.prepare(idsd, posd, ex.to(DEV), mask.to(DEV), total,
                         None if row_shift is None else row_shift.to(DEV))
        gen.prefill(st, W, idsd, posd)
        got.append(st.logits.cpu().clone())
        gxs.append(st.gx.cpu().long())
        gys.append(st.gy.cpu().long())
        for step in range(1, steps):
            st.tok.copy_(tokens[:, S + step - 1].to(DEV))
            Kn.grid_step(st.tok, st.gx, st.gy, st.gio, st.pos, st.counters)
            gen.decode_layers(st, W, want_logits=True)
            if positions is not None:
                assert torch.equal(st.pos.cpu(), positions[:, step - 1])
            got.append(st.logits.cpu().clone())
            gxs.append(st.gx.cpu().long())
            gys.append(st.gy.cpu().long())
    return torch.stack(got, 1), torch.stack(gxs, 1), torch.stack(gys, 1)


@pytest.mark.parametrize("spec_name,rows,max_new,form", [("tiny_cpu", 8, 64, "fp32"),
                                                         ("tiny_cpu", 8, 64, "bf16"),
                                                         ("small_b256", 8, 24, "bf16"),
                                                         ("medium_b128", 2, 64, "bf16"),
                                                         ("large_b64", 2, 64, "bf16")])
def test_config_slice_decode_vs_oracle(spec_name, rows, max_new, form):
    """BASELINE config 0 whole (tiny, 8 prompts of 3 demo pairs of 1-30-sided grids, 64 greedy
    steps, a cache of S_pad + 64 slots) and slices of configs 2-4 at their real shapes (the
    parity harness's config-2 slice is 8 rows; configs 3 and 4 take 2 rows each so that the fp32
    CPU oracle finishes in seconds): the preset under the reference's initialisation
    (torch.manual_seed(0)) in the config's form -- config 0 as the reference runs it, fp32 with
    its weights unrounded (the fp32 form), and also as a bf16 model; configs 2-4 bf16 -- the
    oracle on the same weights in fp32, prompts of the config's workload spanning its lengths,
    left-padded, the config's cache size.  The decode path itself is teacher-forced through the
    oracle's tokens -- grid step, K2 + decode attention over the static cache, head -- and every
    step's logits must lie within 2e-2 max-abs of the oracle's (the prefill's lengths-1 logits
    included), every argmax difference a near-tie and >= 99.5% of them equal; the free-running
    greedy tokens of generate_output (HIP graph) must agree on >= 99.5% of positions, any
    divergence a near-tie."""
    from mdlarc_scale_amd import generate_output
    from mdlarc_scale_amd.workload import SPECS, build_prompts, left_pad

    spec = SPECS[spec_name]
    prompts = build_prompts(spec)
    order = sorted(range(len(prompts)), key=lambda i: len(prompts[i]))
    sl = [prompts[order[round(k * (len(order) - 1) / max(rows - 1, 1))]] for k in range(rows)]
    ids, pos, mask = left_pad(sl)
    B, S = ids.shape
    slots = spec.cache_slots or S + max_new          # config 0 names no cache size
    m, state = _preset_model(spec.preset, form, max_seq_len=slots)
    om = _oracle_of(m, state)
    ex = torch.arange(B) * 3
    tr = rp.generate_output(om, ids, pos, ex, mask, max_new)
    g = len(tr.step_logits)
    ref = torch.stack(tr.step_logits, 1)

    # teacher-forced decode through the product's decode path (eager launches, same kernels)
    # in a cache of the config's size (configs 2-4; config 0: S_pad + 64)
    got, _, _ = _teacher_forced_decode(m, ids, pos, ex, mask, tr.tokens, g, slots,
                                       positions=torch.stack(tr.step_positions, 1))
    err = (got - ref).abs().max().item()
    with torch.no_grad():
        out = generate_output(m, ids.to(DEV), pos.to(DEV), ex.to(DEV),
                              attention_mask=mask.to(DEV), max_new_tokens=max_new).cpu()
    n = min(out.shape[1], tr.tokens.shape[1])
    agree = (out[:, S:n] == tr.tokens[:, S:n]).float().mean().item()
    print(f"{spec_name} {form} slice (prompts {[len(p) for p in sl]}): teacher-forced decode "
          f"logits max-abs {err:.3e} over {g} steps, free-running agreement {agree:.4f}")
    assert err <= 2e-2
    _near_tie_ok(ref, got.argmax(-1), ref.argmax(-1), err)
    assert agree >= 0.995 or _first_divergence_is_tie(out, tr, S, err)


def test_config2_full_batch_decode_vs_oracle():
    """BASELINE config 2 at its production launch shape: all 256 rows, the 2,048-slot cache, one
    decode-attention work item per (row, head) with no split combine, rows dispatched longest
    first.  After the GPU prefill the cache is copied to the host (bf16 -> fp32) and the fp32
    oracle decodes 4 steps from it; the product's decode path, teacher-forced through the
    oracle's tokens, gives logits within 2e-2 max-abs at every step (every argmax difference a
    near-tie), and the captured greedy step replayed from the same prefill state gives the
    oracle's free-running tokens or a near-tie at each row's first divergence."""
    from mdlarc_scale_amd import kernels as Kn
    from mdlarc_scale_amd.data import END_TOKEN_ID
    from mdlarc_scale_amd.engine import engine_for
    from mdlarc_scale_amd.inference import Generator
    from mdlarc_scale_amd.workload import SPECS, build_prompts, left_pad

    spec = SPECS["small_b256"]
    ids, pos, mask = left_pad(build_prompts(spec))
    B, S = ids.shape
    total = spec.cache_slots
    n_steps = 4
    m, state = _preset_model("small", "bf16", max_seq_len=total)   # config 2 is a bf16 model
    c = m.config
    ex = torch.arange(32).repeat_interleave(8)
    eng, gen = engine_for(m), Generator(m)
    idsd, posd, maskd, exd = ids.to(DEV), pos.to(DEV), mask.to(DEV), ex.to(DEV)
    with torch.no_grad():
        W = eng.packed(torch.device(DEV))
        st = gen.prepare(idsd, posd, exd, maskd, total)
        gen.prefill(st, W, idsd, posd)
        torch.cuda.synchronize()
        # the production launch shape: one work item per (row, head), no workspace, longest
        # rows (smallest kv_start) first
        assert st.split_len >= total and st.ws is None
        assert Kn.attn_decode_workspace_bytes(B, c.n_heads, total, st.split_len) == 0
        ks = st.kv_start.cpu()
        assert bool((ks[st.order.cpu().long()].diff() >= 0).all())
        print(f"config 2 full batch: B={B} S={S} slots={total} split_len={st.split_len}",
              flush=True)
        cache = st.cache.cache[..., :S + n_steps, :].cpu().float()
        tok0, gx0, gy0, gio0 = st.tok.cpu(), st.gx.cpu(), st.gy.cpu(), st.gio.cpu()
        pmask = st.pmask.cpu().bool()

    # fp32 oracle: 4 greedy decode steps from the GPU's prefill cache
    om = rp.OracleModel(rp.OracleConfig(c.d_model, c.n_heads, c.n_layers, c.d_ff,
                                        c.num_examples, c.max_seq_len), state)
    grid = rp.GridState(gx0, gy0, gio0)
    key_mask = torch.ones(B, S + n_steps, dtype=torch.bool)
    key_mask[:, :S] = pmask
    toks, ref, positions = [tok0], [], []
    for step in range(n_steps):
        p_ = grid.update(toks[-1])
        positions.append(p_)
        lg = om.decode_step(toks[-1], p_, ex, cache, S + step, key_mask[:, :S + step + 1])
        ref.append(lg)
        toks.append(lg.argmax(-1))
    ref = torch.stack(ref, 1)
    del cache

    # teacher-forced: the product's decode path fed the oracle's input tokens
    got = []
    with torch.no_grad():
        for step in range(n_steps):
            st.tok.copy_(toks[step].to(DEV))
            Kn.grid_step(st.tok, st.gx, st.gy, st.gio, st.pos, st.counters)
            gen.decode_layers(st, W, want_logits=True)
            assert torch.equal(st.pos.cpu(), positions[step])
            got.append(st.logits.cpu().clone())
    got = torch.stack(got, 1)
    err = (got - ref).abs().max().item()
    assert err <= 2e-2
    _near_tie_ok(ref, got.argmax(-1), ref.argmax(-1), err)

    # free-running: the captured greedy step (the bench's and generate_output's launch) from a
    # fresh prefill of the same batch
    with torch.no_grad():
        st2 = gen.prepare(idsd, posd, exd, maskd, total)
        gen.prefill(st2, W, idsd, posd)
        assert torch.equal(st2.tok.cpu(), tok0)
        Kn.decode_commit(st2.tok, st2.out_ids, S, None, st2.finish, S, END_TOKEN_ID)
        gen.greedy_step(st2, W, True)
        graph = gen.capture_greedy(st2, W, True)
        for _ in range(n_steps - 1):
            graph.replay()
        torch.cuda.synchronize()
        free = st2.out_ids[:, S + 1:S + 1 + n_steps].cpu()
    want = torch.stack(toks[1:], 1)
    agree = (free == want).float().mean().item()
    print(f"config 2 full batch: teacher-forced decode logits max-abs {err:.3e} over {n_steps} "
          f"steps x {B} rows, free-running agreement {agree:.4f}")
    for b in range(B):
        d = (free[b] != want[b]).nonzero()
        if len(d):
            t = int(d[0])
            top = ref[b, t].topk(2).values
            assert (top[0] - top[1]).item() <= 2 * err, f"row {b} step {t}"


def _micro_model(stop_model: bool, form: str):
    """The micro model of the augmentation fixture (bf16-rounded weights) on the GPU -- an fp32
    model as the reference ran it ("fp32"), or converted to bf16 ("bf16", exact) -- and its
    oracle twin on the same weights."""
    from mdlarc_scale_amd import TinyTransformer, TransformerConfig
    from tests.golden_io import augment_weights

    c, w = augment_weights(stop_model)
    m = TinyTransformer(TransformerConfig(d_model=c.d_model, n_heads=c.n_heads,
                                          n_layers=c.n_layers, d_ff=c.d_ff,
                                          num_examples=c.num_examples,
                                          max_seq_len=c.max_seq_len, dropout=0.0))
    m.load_state_dict(w, strict=True)
    if form == "bf16":
        m = m.to(torch.bfloat16)
    return m.to(DEV).eval(), rp.OracleModel(c, w)


@pytest.mark.parametrize("form", FORMS)
def test_constrained_greedy_vs_oracle(form, monkeypatch):
    """Greedy decoding under palette / shape / disallow constraints (src/inference.py:285-364,
    :572, :609) against the oracle, whose constraint rule the reference's own outputs pin bit for
    bit: the constraints fused into the head kernels of the captured step and the host-launched
    path give the same tokens; teacher-forced through the oracle's tokens, the decode path's
    logits lie within 2e-2 of the oracle's (bf16 form: 2e-2 * max|logit|; the micro model's
    logits reach |28|), and with the oracle's rule applied on the decode path's own grid state
    every constrained argmax agrees or is a near-tie (top-2 gap <= 2x the error); free-running
    agreement >= 99.5% or a near-tie at each row's first divergence.  The constraints change the
    tokens."""
    from mdlarc_scale_amd import inference as inf

    m, om = _micro_model(False, form)
    rng = np.random.default_rng(9)
    ids, pos, mask = _left_pad(_random_prompts(rng, 6, 2, 1, 4))
    B, S = ids.shape
    g = torch.Generator().manual_seed(9)
    pal = torch.rand(6, 10, generator=g) < 0.5
    pal[0] = True
    shape = torch.randint(1, 5, (6, 2), generator=g)
    shape[1] = -1
    ex = torch.tensor([0, 1, 2, 3, 0, 1])
    max_new = 40
    ocons = rp.OracleConstraints(palette_mask=pal, target_shape=shape)
    tr = rp.generate_output(om, ids, pos, ex, mask, max_new, True, ocons)
    cons = inf.DecodingConstraints(palette_mask=pal.to(DEV), target_shape=shape.to(DEV))
    outs = {}
    for fused in (True, False):
        monkeypatch.setattr(inf, "FUSED_CONSTRAINTS", fused)
        with torch.no_grad():
            outs[fused] = inf.generate_output(m, ids.to(DEV), pos.to(DEV), ex.to(DEV),
                                              mask.to(DEV), max_new_tokens=max_new,
                                              constraints=cons).cpu()
    with torch.no_grad():
        free = inf.generate_output(m, ids.to(DEV), pos.to(DEV), ex.to(DEV), mask.to(DEV),
                                   max_new_tokens=max_new).cpu()
    assert torch.equal(outs[True], outs[False])
    n = min(free.shape[1], outs[True].shape[1])
    assert not torch.equal(free[:, :n], outs[True][:, :n])

    steps = len(tr.step_logits)
    raw, gx, gy = _teacher_forced_decode(m, ids, pos, ex, mask, tr.tokens, steps, S + max_new,
                                         positions=torch.stack(tr.step_positions, 1))
    ref_raw = torch.stack(tr.raw_logits, 1)
    ref = torch.stack(tr.step_logits, 1)
    err = (raw - ref_raw).abs().max().item()
    scale = ref_raw.abs().max().item()
    got = torch.stack([rp.apply_logit_constraints(raw[:, t].clone(), gx[:, t], gy[:, t], ocons)
                       for t in range(steps)], 1)
    out = outs[True]
    n = min(out.shape[1], tr.tokens.shape[1])
    agree = (out[:, S:n] == tr.tokens[:, S:n]).float().mean().item()
    print(f"constrained micro ({form}): teacher-forced logits max-abs {err:.3e} (max |logit| "
          f"{scale:.1f}), free-running agreement {agree:.4f}")
    assert err <= (2e-2 if form == "fp32" else 2e-2 * scale)
    # the bf16 form on the sharp micro model: near-ties only, as in the augmentation test
    _near_tie_ok(ref, got.argmax(-1), ref.argmax(-1), err, 0.995 if form == "fp32" else None)
    assert agree >= 0.995 or _first_divergence_is_tie(out, tr, S, err)


@pytest.mark.parametrize("form", FORMS)
def test_packed_prefill_equals_padded(form, monkeypatch):
    """Prefill over the packed token list (left padding left out, the padding tokens that the
    lengths-1 index names appended) against prefill over the whole padded batch: first-step logits
    equal to GEMM rounding (the GEMMs see another row count), every valid cache slot equal to one
    bf16 ulp, the same first token unless the two best logits are tied to that rounding.  Half
    the rows are shorter than their padding, so their logits come from extra rows.  (Generation
    on the packed path is checked against the oracle and the golden traces.)"""
    from mdlarc_scale_amd import inference as inf

    m, _ = _preset_model("small", form, seed=4, max_seq_len=2048)
    rng = np.random.default_rng(44)
    prompts = _random_prompts(rng, 4, 3, 3, 9) + _random_prompts(rng, 4, 1, 1, 2)
    ids, pos, mask = _left_pad(prompts)
    ids, pos, mask = ids.to(DEV), pos.to(DEV), mask.to(DEV)
    B, S = ids.shape
    ex = torch.arange(B, device=DEV)
    kv = (S - mask.sum(1)).cpu()
    assert int(((S - kv) * 2 < S).sum()) >= 2        # rows whose lengths-1 index is padding
    res = {}
    for packed in (True, False):
        monkeypatch.setattr(inf, "PACKED_PREFILL", packed)
        gen = inf.Generator(m)
        with torch.no_grad():
            W = gen.eng.packed(ids.device)
            st = gen.prepare(ids, pos, ex, mask, S + 8)
            gen.prefill(st, W, ids, pos)
        torch.cuda.synchronize()
        res[packed] = (st.logits.cpu(), st.tok.cpu(), st.cache)
    lp, tp, cp = res[True]
    lq, tq, cq = res[False]
    err = (lp - lq).abs().max().item()
    print(f"packed vs padded prefill: logits max-abs {err:.3e}")
    assert err <= 1e-3
    _near_tie_ok(lq, tp, tq, err, min_agree=None)
    for li in range(m.config.n_layers):
        for a, b in zip(cp.layer(li), cq.layer(li)):
            for r in range(B):
                k0 = int(kv[r])
                x, y = a[r, :, k0:S].float(), b[r, :, k0:S].float()
                # one bf16 ulp (bf16 form) / fp32 rounding of the GEMMs (fp32 form)
                tol = 2 ** -7 if form == "bf16" else 1e-5
                assert bool(((x - y).abs() <= tol * y.abs() + 1e-6).all())


def test_decode_forms_agree(monkeypatch):
    """The decode step on K5 with the norms, SwiGLU and residual adds fused (five launches per
    layer, tiled x) against the separate-kernel form (hipBLASLt, add+RMSNorm, K3; row-major):
    the same greedy tokens for a ragged batch whose size is not a multiple of 16 (the tile
    layout's padding rows), and the logits of the first decode step equal to GEMM rounding
    (generation replays a captured graph; the logits come from the host-launched step)."""
    from mdlarc_scale_amd import inference as inf
    from mdlarc_scale_amd import kernels as K

    m, _ = _preset_model("small", "bf16", seed=7, max_seq_len=2048)   # the forms are bf16's
    rng = np.random.default_rng(77)
    prompts = _random_prompts(rng, 9, 2, 2, 6) + _random_prompts(rng, 4, 1, 1, 3)
    ids, pos, mask = _left_pad(prompts)
    ids, pos, mask = ids.to(DEV), pos.to(DEV), mask.to(DEV)
    B = ids.shape[0]
    assert B % 16 != 0
    ex = torch.arange(B, device=DEV)
    out, logits = {}, {}
    for tiled in (True, False):
        monkeypatch.setattr(inf, "DECODE_TILED", tiled)
        with torch.no_grad():
            out[tiled] = inf.generate_output(m, ids, pos, ex, attention_mask=mask,
                                             max_new_tokens=40, stop_on_end=False).cpu()
            gen = inf.Generator(m)
            W = gen.eng.packed(ids.device)
            st = gen.prepare(ids, pos, ex, mask, ids.shape[1] + 4)
            assert st.sc.tiled == tiled
            gen.prefill(st, W, ids, pos)
            # the host-launched step: position of the prefill's token, then the layers
            K.grid_step(st.tok, st.gx, st.gy, st.gio, st.pos, st.counters)
            gen.decode_layers(st, W, want_logits=True)
            torch.cuda.synchronize()
            logits[tiled] = st.logits.cpu()
    err = (logits[True] - logits[False]).abs().max().item()
    agree = (out[True] == out[False]).float().mean().item()
    print(f"decode forms: first decode step logits max-abs {err:.3e}, token agreement {agree:.4f}")
    assert err <= 1e-3
    assert torch.equal(out[True], out[False])


@pytest.mark.parametrize("decode_tiled", [True, False])
def test_prompt_path_without_k6_vs_oracle(decode_tiled, monkeypatch):
    """The bf16 form's prompt path for model shapes K6 does not take (d_model above 2048, widths
    that are not multiples of 32): hipBLASLt on [W | W], then qkv_rope_cache(_packed) with the
    log2(e) q scale, K4a + K4c, add_rmsnorm and K3 as separate launches.  Forced on the tiny
    preset (bf16) by reporting every shape as outside K6; with decode_tiled False the decode step
    also takes its separate-kernel form.  forward and generate_output against the oracle at the
    2e-2 bar, argmax differences near-ties."""
    from mdlarc_scale_amd import engine
    from mdlarc_scale_amd import inference as inf

    monkeypatch.setattr(engine, "prompt_gemms_fused", lambda d_model, d_ff: False)
    monkeypatch.setattr(inf, "DECODE_TILED", decode_tiled)
    m, state = _preset_model("tiny", "bf16", seed=5)
    rng = np.random.default_rng(55)
    ids, pos, mask = _left_pad(_random_prompts(rng, 4, 3, 1, 7))
    ex = torch.tensor([2, 0, 11, 40])
    sc = engine.Scratch.for_prompt(8, m.config, torch.device(DEV), False)
    assert not sc.fused and not sc.tiled                 # the hipBLASLt prompt form runs
    ref = _oracle_of(m, state).forward(ids, pos, ex, mask, True)
    got = _fwd(m, ids, pos, ex, mask)
    err = (got - ref)[mask].abs().max().item()
    print(f"prompt path without K6: forward logits max-abs {err:.3e}")
    assert err <= 2e-2
    _compare_with_oracle(m, state, ids, pos, ex, mask, 32, f"no-K6 decode_tiled={decode_tiled}")


@pytest.mark.parametrize("spec_name,rows,drops", [
    ("small_b256", 8, ["qkv", "out", "gate_up", "down", "qkv+out"]),
    ("medium_b128", 2, ["qkv", "out", "qkv+out"]), ("large_b64", 2, ["qkv", "out", "qkv+out"])])
def test_prompt_projection_lo_terms(monkeypatch, spec_name, rows, drops):
    """What each prompt projection's lo term is worth at configs 2-4's real prompt lengths (the
    parity harness's slices: 8 rows of config 2, 2 of configs 3 and 4; bf16): the prompt path's
    projections take their
    split inputs through gemm_f32 when K6 is off, so zeroing the lo half of one projection's
    input there drops exactly that projection's lo product (qkv, out, gate/up or down; the
    decode path is untouched, and reads the cache the prefill wrote).  Prints each variant's
    teacher-forced decode error against the fp32 oracle; asserts only that the split forward
    keeps the 2e-2 bar and that each variant changes the logits (the drop took effect).
    Measured: qkv or out alone 7.3e-3 / 8.0e-3 at config 2 and 6.1e-3 / 6.7e-3 at config 3, but
    1.2e-2 / 1.3e-2 at config 4's 5,000-token prompts (split: 4.8e-3 / 4.4e-3 / 6.0e-3), so the
    engine keeps both parts on every projection."""
    from mdlarc_scale_amd import engine
    from mdlarc_scale_amd.workload import SPECS, build_prompts, left_pad

    spec = SPECS[spec_name]
    prompts = build_prompts(spec)
    order = sorted(range(len(prompts)), key=lambda i: len(prompts[i]))
    sl = [prompts[order[round(k * (len(order) - 1) / (rows - 1))]] for k in range(rows)]
    ids, pos, mask = left_pad(sl)
    B, S = ids.shape
    max_new = 24
    m, state = _preset_model(spec.preset, "bf16", max_seq_len=spec.cache_slots)
    om = _oracle_of(m, state)
    ex = torch.arange(B) * 3
    tr = rp.generate_output(om, ids, pos, ex, mask, max_new)
    g = len(tr.step_logits)
    ref = torch.stack(tr.step_logits, 1)

    monkeypatch.setattr(engine, "prompt_gemms_fused", lambda d_model, d_ff: False)
    real = engine.gemm_f32
    names = ["qkv", "out", "gate_up", "down"]   # the prompt path's gemm_f32 calls, per layer
    errs, outs = {}, {}
    for drop in [None] + drops:
        calls = [0]

        def gemm(a, w2, out, drop=drop, calls=calls):
            if drop is not None and names[calls[0] % 4] in drop.split("+"):
                a = a.clone()
                a[:, a.shape[1] // 2:] = 0           # the lo half of the split input
            calls[0] += 1
            return real(a, w2, out)

        monkeypatch.setattr(engine, "gemm_f32", gemm)
        got, _, _ = _teacher_forced_decode(m, ids, pos, ex, mask, tr.tokens, g,
                                           spec.cache_slots)
        assert calls[0] == 4 * m.config.n_layers
        errs[drop] = (got - ref).abs().max().item()
        outs[drop] = got
    print(f"{spec_name} slice (prompts {[len(p) for p in sl]}), prompt projection lo term "
          "dropped -> teacher-forced decode max-abs: "
          + ", ".join(f"{k or 'none'} {v:.3e}" for k, v in errs.items()))
    assert errs[None] <= 2e-2
    for name in drops:
        assert (outs[name] - outs[None]).abs().max().item() > 0


def test_prompt_mlp_single_part_vs_oracle(monkeypatch):
    """The prompt MLP with the lo term dropped (engine.PROMPT_GATE_UP_PARTS and
    PROMPT_DOWN_PARTS at 1: gate / up on bf16(ln2(x)), h stored and read as hi alone) -- an
    option the engine does not take by default.  The small preset's bf16 forward stays inside
    the 2e-2 bar (about 1e-2 measured), and moves away from the default split forward (the
    option takes effect)."""
    from mdlarc_scale_amd import engine, kernels

    m, state = _preset_model("small", "bf16", seed=9)
    rng = np.random.default_rng(91)
    ids, pos, mask = _left_pad(_random_prompts(rng, 4, 3, 1, 8))
    ex = torch.tensor([3, 0, 9, 27])
    ref = _oracle_of(m, state).forward(ids, pos, ex, mask, True)
    split_fwd = _fwd(m, ids, pos, ex, mask)
    monkeypatch.setattr(engine, "PROMPT_GATE_UP_PARTS", 1)
    monkeypatch.setattr(engine, "PROMPT_DOWN_PARTS", 1)
    sc = engine.Scratch.for_prompt(40, m.config, torch.device(DEV), False)
    assert sc.fused and sc.h.numel() == kernels.tile_rows(40) * m.config.d_ff
    got = _fwd(m, ids, pos, ex, mask)
    err = (got - ref)[mask].abs().max().item()
    err_split = (split_fwd - ref)[mask].abs().max().item()
    print(f"prompt MLP single part: forward max-abs {err:.3e} (split {err_split:.3e})")
    assert err <= 2e-2
    assert (got - split_fwd)[mask].abs().max().item() > 1e-3


@pytest.mark.parametrize("form", FORMS)
def test_checkpoint_ingest_on_gpu_vs_oracle(tmp_path, form):
    """Checkpoint ingest (src/eval.py:881-951) onto the GPU, where the weights are packed and
    tiled at load: a reference training checkpoint (the keys of src/train.py:938-950; perturbed
    norm gains and biases, so those paths carry weight) loaded with
    load_model_from_checkpoint(path, "cuda", return_task_id_map=True) generates and forwards
    like the fp32 oracle on the checkpoint's weights (2e-2, near-tie rule).  "bf16" converts the
    loaded model with .to(bfloat16), as a bf16 configuration runs it.  Then one step of the
    example-embedding adaptation of src/eval.py:159-205 -- Adam on example_embed.weight through
    the autograd forward, and the weight decay written through .data -- and the next generation
    follows the edited rows: it matches the oracle on the edited weights, and its logits move."""
    from dataclasses import asdict

    from mdlarc_scale_amd import create_tiny_model
    from mdlarc_scale_amd.checkpoint import load_model_from_checkpoint

    torch.manual_seed(11)
    src = create_tiny_model(dropout=0.0, max_seq_len=1024)
    g = torch.Generator().manual_seed(11)
    with torch.no_grad():
        for n, p in src.named_parameters():
            if n.endswith("ln1.weight") or n.endswith("ln2.weight") or n == "ln_f.weight":
                p.copy_(1 + 0.1 * torch.randn(p.shape, generator=g))
            elif n.endswith(".bias"):
                p.copy_(0.02 * torch.randn(p.shape, generator=g))
            elif n == "example_embed.weight":      # trained example rows, not the N(0, 0.02) init
                p.copy_(0.5 * torch.randn(p.shape, generator=g))
    ckpt = {"model_state": src.state_dict(), "model_config": asdict(src.config),
            "optimizer_state": {}, "scheduler_state": {}, "epoch": 2, "global_step": 500,
            "config": {"model_size": "tiny"}, "metrics": {"loss": 0.7},
            "rng_state": {"python": None, "numpy": np.random.get_state(),
                          "torch": torch.get_rng_state()},
            "task_id_to_example_id": {"task_a": 3, "task_b": 7, "task_c": 1023}}
    path = tmp_path / "checkpoint.pt"
    torch.save(ckpt, path)
    m, task_map = load_model_from_checkpoint(path, DEV, return_task_id_map=True)
    assert task_map == ckpt["task_id_to_example_id"] and not m.training
    assert next(m.parameters()).is_cuda
    if form == "bf16":
        m = m.to(torch.bfloat16)
    state = {k: v.float().cpu().clone() for k, v in m.state_dict().items()}
    for k, v in src.state_dict().items():                # the file's weights, as loaded
        assert torch.equal(state[k], v.to(next(m.parameters()).dtype).float()), k
    rng = np.random.default_rng(111)
    ids, pos, mask = _left_pad(_random_prompts(rng, 3, 2, 1, 7))
    ex = torch.tensor([task_map["task_a"], task_map["task_b"], task_map["task_c"]])
    _compare_with_oracle(m, state, ids, pos, ex, mask, 32, f"checkpoint {form}")
    before = _fwd(m, ids, pos, ex, mask)

    # one adaptation step of example row 3 (src/eval.py:170-203).  The bf16 model writes the
    # adapted row through .data instead of taking the Adam step: its autograd forward would run
    # bf16 batched products on the GPU, which are kept out of every GPU run here.
    ex_id, lr, wd = task_map["task_a"], 0.05, 0.01
    if form == "fp32":
        params = list(m.parameters())
        for p in params:
            p.requires_grad_(False)
        m.example_embed.weight.requires_grad_(True)
        opt = torch.optim.Adam([m.example_embed.weight], lr=lr)
        opt.zero_grad()
        sel = ex == ex_id
        logits = m(ids[sel].to(DEV), pos[sel].to(DEV), example_ids=ex[sel].to(DEV),
                   attention_mask=mask[sel].to(DEV))
        logits.logsumexp(-1).mean().backward()
        opt.step()
        for p in params:
            p.requires_grad_(True)
    else:
        delta = lr * torch.randn(m.config.d_model, generator=g).sign()
        m.example_embed.weight.data[ex_id] += delta.to(DEV, torch.bfloat16)
    with torch.no_grad():
        m.example_embed.weight.data[ex_id].mul_(1.0 - lr * wd)
    state2 = {k: v.float().cpu().clone() for k, v in m.state_dict().items()}
    moved = (state2["example_embed.weight"] - state["example_embed.weight"]).abs().amax(1)
    assert moved[ex_id] > 0.01 and int((moved > 0).sum()) == 1
    _compare_with_oracle(m, state2, ids, pos, ex, mask, 32, f"checkpoint {form} after TTA")
    after = _fwd(m, ids, pos, ex, mask)
    shift = (after - before).abs().amax((1, 2))
    print(f"checkpoint {form}: logit shift per row after the edit {shift.tolist()}")
    assert shift[0] > 0.1 and shift[1] == 0 and shift[2] == 0


@pytest.mark.parametrize("form", FORMS)
def test_reference_private_step_functions_vs_oracle(form):
    """_prefill, _decode_step and _get_decode_fn with the reference's arguments
    (src/inference.py:383-479) -- a decode loop written against them, as the body of the
    reference's generate_output is, over a StaticKVCache in the model's dtype, teacher-forced
    through the oracle's tokens and positions: logits at every step within 2e-2 of the oracle's
    (plus one bf16 ulp of the logit for a bf16 model, whose step functions return bf16 logits as
    the reference's do); the cache advances as the reference's does."""
    from mdlarc_scale_amd import inference as inf

    m, state = _preset_model("tiny", form, seed=8)
    rng = np.random.default_rng(88)
    ids, pos, mask = _left_pad(_random_prompts(rng, 3, 2, 1, 6))
    ex = torch.tensor([1, 2, 3])
    B, S = ids.shape
    steps = 12
    tr = rp.generate_output(_oracle_of(m, state), ids, pos, ex, mask, steps)
    g = len(tr.step_logits)
    c = m.config
    dt = next(m.parameters()).dtype
    cache = inf.StaticKVCache(B, S + steps, c.n_layers, c.n_heads, 64, torch.device(DEV), dt)
    full = torch.cat([mask, torch.ones(B, steps, dtype=torch.bool)], 1).to(DEV)
    decode = inf._get_decode_fn(True)
    with torch.no_grad():
        lg = inf._prefill(m, ids.to(DEV), pos.to(DEV), ex.to(DEV), cache, mask.to(DEV))
        assert lg.shape == (B, 1, 14) and lg.dtype == dt and cache.seq_len == S
        got = [lg[:, 0].float().cpu()]
        for t in range(1, g):
            tok = tr.tokens[:, S + t - 1:S + t]
            p_ = tr.step_positions[t - 1][:, None]
            lg = decode(m, tok.to(DEV), p_.to(DEV), ex.to(DEV), cache, full[:, :S + t])
            assert cache.seq_len == S + t
            got.append(lg[:, 0].float().cpu())
    got = torch.stack(got, 1)
    ref = torch.stack(tr.step_logits, 1)
    err = (got - ref).abs()
    bound = 2e-2 + (2 ** -8 * ref.abs() if form == "bf16" else 0)
    print(f"reference step functions ({form}): logits max-abs {err.max().item():.3e} over {g} "
          f"steps")
    assert bool((err <= bound).all())
    # the argmax of bf16-rounded logits flips between near-tied tokens: near-ties only (the
    # 99.5% agreement of the decode path is pinned by the fp32-logit tests above)
    _near_tie_ok(ref, got.argmax(-1), ref.argmax(-1), err.max().item(),
                 0.995 if form == "fp32" else None)
