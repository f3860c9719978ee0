"""Pin the CPU oracle before trusting it (CPU only).

1. Golden vectors written from the reference itself (tests/golden/make_golden.py): forward
   logits, generate_output tokens / per-step logits / decode positions on a left-padded ragged
   batch, stop-on-END, grid-state traces, initial-state derivation, colour permutations.
2. Closed forms and invariants in fp64 for the elementary ops, chosen so that a dropped term, a
   wrong sign or a transposed index fails.
"""

import math

import numpy as np
import pytest
import torch

from oracle import data_format as odf
from oracle import reference_path as rp
from tests.golden_io import augment_weights, constraint_cases, load_augment, load_e2e

# ------------------------------------------------------------------ golden end-to-end vectors


@pytest.mark.parametrize("name", ["e2e_micro", "e2e_micro_stop"])
def test_forward_matches_reference_golden(name):
    fx = load_e2e(name)
    m = rp.OracleModel(fx.cfg, fx.weights)
    got = m.forward(fx.ids, fx.pos, fx.ex_ids, fx.mask, True)
    assert (got - fx.fwd_logits).abs().max().item() < 1e-4


@pytest.mark.parametrize("name", ["e2e_micro", "e2e_micro_stop"])
def test_generate_matches_reference_golden(name):
    fx = load_e2e(name)
    m = rp.OracleModel(fx.cfg, fx.weights)
    tr = rp.generate_output(m, fx.ids, fx.pos, fx.ex_ids, fx.mask, fx.max_new)
    assert torch.equal(tr.tokens, fx.gen)
    assert (torch.stack(tr.step_logits, 1) - fx.step_logits).abs().max().item() < 1e-4
    if fx.step_pos.shape[1]:
        assert torch.equal(torch.stack(tr.step_positions, 1), fx.step_pos)
    # no mask, no example ids: example id defaults to 0
    p = fx.single_prompt
    pos = torch.from_numpy(odf.compute_positions_3d(p.tolist()))[None]
    tr1 = rp.generate_output(m, p[None], pos, None, None, 12)
    assert torch.equal(tr1.tokens, fx.single_gen)


def test_stop_fixture_really_stops_early():
    fx = load_e2e("e2e_micro_stop")
    S = fx.ids.shape[1]
    gen = fx.gen[:, S:]
    assert gen.shape[1] < fx.max_new                       # broke before max_new
    assert all((row == 13).any() for row in gen)           # every row emitted END
    assert (gen[:, -1] == 13).any()                        # last row finished on the last step


def test_left_pad_quirk_is_exercised():
    """Row 0 is short enough that index lengths-1 lands inside its left padding."""
    fx = load_e2e("e2e_micro")
    n = fx.mask.sum(1)
    S = fx.ids.shape[1]
    assert (n - 1 < S - n).any()                           # quirk index inside the pad
    assert ((n - 1 >= S - n) & (n < S)).any()              # quirk index mid-prompt
    assert (n == S).any()


def _oracle_constraints(c):
    return rp.OracleConstraints(palette_mask=c["palette"], target_shape=c["shape"],
                                palette_penalty=c["palette_penalty"],
                                shape_penalty=c["shape_penalty"], disallow_tokens=c["disallow"])


def test_constraints_match_reference_golden():
    """The oracle's constraint rule returns the reference's logits bit for bit on every case
    (broadcast rows, mismatched batches, rows without a shape, x == w / y == h, the early
    return on a grid-state batch mismatch, a huge penalty)."""
    cases = constraint_cases()
    assert len(cases) >= 9
    for i, c in enumerate(cases):
        got = rp.apply_logit_constraints(c["logits"].clone(), c["gx"], c["gy"],
                                         _oracle_constraints(c))
        assert torch.equal(got, c["out"]), f"case {i}"
    # the fixture exercises every branch: each penalty changes some logit somewhere
    changed = [(c["out"] != c["logits"]) for c in cases]
    assert any(ch[:, :10].any() for ch in changed)          # palette / shape on colours
    assert any(ch[:, 11].any() for ch in changed)           # shape on NEWLINE
    assert any(torch.equal(c["out"][:, :10], c["logits"][:, :10]) and c["palette"] is not None
               for c in cases)                              # a skipped (mismatched) palette


def test_constraint_rule_plants_fail():
    """Plausible mistakes in the rule (here: the row-complete test inverted) change the result
    on the fixture, so the bit-exact comparison above would catch them."""
    c = constraint_cases()[0]
    good = rp.apply_logit_constraints(c["logits"].clone(), c["gx"], c["gy"],
                                      _oracle_constraints(c))
    bad = rp.apply_logit_constraints(c["logits"].clone(), c["gx"] - 1, c["gy"],
                                     _oracle_constraints(c))
    assert not torch.equal(good, bad)


@pytest.mark.parametrize("r", range(7))
def test_augmentations_match_reference_golden(r):
    """The oracle's augmentation caller reproduces the reference's runs: per variant the token
    stream its prediction is decoded from, its generated tokens (the chunk's stop step) and the
    dihedral / permutation labels."""
    from oracle import augment as oa

    fx = load_augment()
    run = fx.runs[r]
    cfg, w = augment_weights(run.stop_model)
    m = rp.OracleModel(cfg, w)
    tr = oa.predict_with_augmentations(
        m, fx.task, 0, example_id=fx.example_id, num_color_perms=fx.num_color_perms,
        max_output_tokens=fx.max_new, constrain_decoding=run.constrain, batched=run.batched,
        max_batch_size=run.chunk, decode=lambda toks: tuple(toks))
    assert [(p[1], p[2]) for p in tr.predictions] == run.aug
    assert tr.generated == run.gen
    assert [p[0] for p in tr.predictions] == run.streams


def test_augmentation_grids_match_reference_golden():
    from oracle import augment as oa

    fx = load_augment()
    cfg, w = augment_weights(True)
    tr = oa.predict_with_augmentations(rp.OracleModel(cfg, w), fx.task, 0,
                                       example_id=fx.example_id,
                                       num_color_perms=fx.num_color_perms,
                                       max_output_tokens=fx.max_new)
    assert [p[0] for p in tr.predictions] == fx.grids


def test_grid_state_matches_reference_golden():
    g = np.load("tests/golden/grid_state.npz")
    gs = rp.GridState(torch.from_numpy(g["x0"]), torch.from_numpy(g["y0"]),
                      torch.from_numpy(g["io0"]))
    trace = [gs.update(torch.from_numpy(g["tokens"][:, s])).numpy()
             for s in range(g["tokens"].shape[1])]
    assert np.array_equal(np.stack(trace, 1), g["positions"])
    fin = np.stack([gs.x.numpy(), gs.y.numpy(), gs.in_output.numpy().astype(np.int64)], 1)
    assert np.array_equal(fin, g["final"])
    ix, iy, io = rp.derive_initial_state(torch.from_numpy(g["p_ids"]),
                                         torch.from_numpy(g["p_pos"]),
                                         torch.from_numpy(g["p_mask"]))
    init = np.stack([ix.numpy(), iy.numpy(), io.numpy().astype(np.int64)], 1)
    assert np.array_equal(init, g["init"])


def test_grid_state_equals_compute_positions_on_streams():
    """Feeding a whole prompt token by token through the updater reproduces
    compute_positions_3d (invariant between the two restatements of one rule)."""
    rng = np.random.default_rng(3)
    for _ in range(20):
        toks = []
        for _pair in range(rng.integers(1, 4)):
            h, w = rng.integers(1, 33, size=2)
            grid = rng.integers(0, 10, size=(h, w)).tolist()
            toks += odf.encode_example(grid, grid)
        ref = odf.compute_positions_3d(toks)
        gs = rp.GridState(torch.zeros(1), torch.zeros(1), torch.zeros(1, dtype=torch.bool))
        got = np.stack([gs.update(torch.tensor([t]))[0].numpy() for t in toks])
        assert np.array_equal(got, ref)


def test_color_perms_match_reference_golden():
    c = np.load("tests/golden/color_perms.npz")
    assert np.array_equal(odf.color_permutations(8, 42), c["p8_42"])
    assert np.array_equal(odf.color_permutations(16, 42), c["p16_42"])
    assert np.array_equal(odf.color_permutations(8, 7), c["p8_7"])


# ------------------------------------------------------------------ closed forms (fp64)

def test_rmsnorm_closed_form():
    w = torch.tensor([1.0, 2.0, 0.5, -1.0], dtype=torch.float64)
    x = torch.tensor([[3.0, 3.0, 3.0, 3.0], [1.0, -1.0, 1.0, -1.0], [2.0, 0.0, 0.0, 0.0]],
                     dtype=torch.float64)
    y = rp.rmsnorm(x, w, 0.0)
    # constant row c: x / |c| ; alternating +-1: unchanged ; single spike 2 at d=4: 2/sqrt(1)=2
    exp = torch.tensor([[1, 2, 0.5, -1], [1, -2, 0.5, 1], [2, 0, 0, 0]], dtype=torch.float64)
    assert torch.allclose(y, exp)
    # eps enters inside the square root
    y2 = rp.rmsnorm(torch.ones(1, 4, dtype=torch.float64), torch.ones(4, dtype=torch.float64), 3.0)
    assert torch.allclose(y2, torch.full((1, 4), 0.5, dtype=torch.float64))
    # scale invariance (eps=0)
    z = torch.randn(5, 64, dtype=torch.float64)
    assert torch.allclose(rp.rmsnorm(z, w.new_ones(64), 0.0), rp.rmsnorm(7.5 * z, w.new_ones(64), 0.0))


def test_silu_swiglu_closed_form():
    a = torch.tensor([-3.0, -0.5, 0.0, 0.5, 3.0], dtype=torch.float64)
    exp = a / (1 + torch.exp(-a))
    assert torch.allclose(rp.silu(a), exp)
    # one-channel SwiGLU with hand-set weights: gate = 2x+b_g, up = -x+b_u, down = 3h+b_d
    w = {"f.fc_gate.weight": torch.tensor([[2.0]], dtype=torch.float64),
         "f.fc_gate.bias": torch.tensor([0.25], dtype=torch.float64),
         "f.fc_up.weight": torch.tensor([[-1.0]], dtype=torch.float64),
         "f.fc_up.bias": torch.tensor([1.0], dtype=torch.float64),
         "f.fc_down.weight": torch.tensor([[3.0]], dtype=torch.float64),
         "f.fc_down.bias": torch.tensor([-0.5], dtype=torch.float64)}
    x = torch.tensor([[0.7]], dtype=torch.float64)
    g = 2 * 0.7 + 0.25
    exp = 3 * (g / (1 + math.exp(-g))) * (-0.7 + 1.0) - 0.5
    assert abs(rp.swiglu_ffn(x, w, "f.").item() - exp) < 1e-12


def _cfg(**kw):
    base = dict(d_model=128, n_heads=2, n_layers=1, d_ff=64)
    base.update(kw)
    return rp.OracleConfig(**base)


def test_rope_split_and_tables():
    assert rp.rope3d_split(64) == (10, 10, 12)
    cfg = _cfg()
    t = rp.rope3d_tables(cfg)
    assert t["cos_x"].shape == (32, 10) and t["cos_z"].shape == (8, 12)
    # inv_freq of axis x = base^(-2j/20): angle at pos 1, pair 1 = 10000^(-0.1)
    assert abs(math.acos(t["cos_x"][1, 1].item()) - 10000 ** -0.1) < 1e-6
    assert abs(math.acos(t["cos_z"][1, 3].item()) - 10000 ** (-6 / 24)) < 1e-6


def test_rope_identity_norm_and_clamp():
    cfg = _cfg()
    tab = {k: v.double() for k, v in rp.rope3d_tables(cfg).items()}
    q = torch.randn(2, 5, 3, 64, dtype=torch.float64)
    zero = torch.zeros(2, 5, 3, dtype=torch.long)
    assert torch.allclose(rp.apply_rope3d(q, zero, tab, cfg), q)          # identity at origin
    pos = torch.randint(0, 40, (2, 5, 3))
    r = rp.apply_rope3d(q, pos, tab, cfg)
    nq = q.unflatten(-1, (32, 2)).norm(dim=-1)
    nr = r.unflatten(-1, (32, 2)).norm(dim=-1)
    assert torch.allclose(nq, nr)                                        # per-pair norm
    big = torch.full((2, 5, 3), 100)
    top = torch.tensor([31, 31, 7]).expand(2, 5, 3)
    assert torch.allclose(rp.apply_rope3d(q, big, tab, cfg), rp.apply_rope3d(q, top, tab, cfg))
    neg = torch.full((2, 5, 3), -4)
    assert torch.allclose(rp.apply_rope3d(q, neg, tab, cfg), q)          # clamps to 0


def test_rope_reduces_to_textbook_1d_on_x_axis():
    """With y = z = 0 dims 20..63 are untouched and dims 0..19 are interleaved RoPE, dim 20."""
    cfg = _cfg()
    tab = {k: v.double() for k, v in rp.rope3d_tables(cfg).items()}
    q = torch.randn(1, 4, 1, 64, dtype=torch.float64)
    xs = torch.tensor([0, 1, 5, 29])
    pos = torch.stack([xs, torch.zeros(4, dtype=torch.long), torch.zeros(4, dtype=torch.long)],
                      -1)[None]
    r = rp.apply_rope3d(q, pos, tab, cfg)
    assert torch.allclose(r[..., 20:], q[..., 20:])
    for s, p in enumerate(xs.tolist()):
        for j in range(10):
            th = p * 10000.0 ** (-2 * j / 20)
            a, b = q[0, s, 0, 2 * j].item(), q[0, s, 0, 2 * j + 1].item()
            assert abs(r[0, s, 0, 2 * j].item() - (a * math.cos(th) - b * math.sin(th))) < 1e-6
            assert abs(r[0, s, 0, 2 * j + 1].item() - (b * math.cos(th) + a * math.sin(th))) < 1e-6


def test_rope_relative_position_property():
    """<R(p)q, R(p')k> depends only on p' - p along each axis (inside the clamp range)."""
    cfg = _cfg()
    tab = {k: v.double() for k, v in rp.rope3d_tables(cfg).items()}
    q = torch.randn(64, dtype=torch.float64).view(1, 1, 1, 64)
    k = torch.randn(64, dtype=torch.float64).view(1, 1, 1, 64)

    def dot(p, pk):
        a = rp.apply_rope3d(q, torch.tensor([[p]]), tab, cfg)
        b = rp.apply_rope3d(k, torch.tensor([[pk]]), tab, cfg)
        return (a * b).sum().item()

    # the angle tables are fp32 (as in the reference), hence the fp32-level tolerance
    assert abs(dot([2, 3, 1], [7, 4, 3]) - dot([10, 20, 2], [15, 21, 4])) < 1e-6
    assert abs(dot([2, 3, 1], [7, 4, 3]) - dot([2, 3, 1], [8, 4, 3])) > 1e-3


def test_attention_brute_force_and_zero_rows():
    torch.manual_seed(0)
    B, H, S, hd = 2, 2, 7, 64
    q, k, v = (torch.randn(B, H, S, hd, dtype=torch.float64) for _ in range(3))
    mask = torch.ones(B, S, dtype=torch.bool)
    mask[0, :3] = False
    mask[1, 4] = False
    out = rp.attention(q, k, v, mask, causal=True)
    for b in range(B):
        for h in range(H):
            for i in range(S):
                keys = [j for j in range(S) if j <= i and mask[b, j]]
                if not keys:
                    assert torch.all(out[b, h, i] == 0)
                    continue
                s = torch.stack([q[b, h, i] @ k[b, h, j] / 8.0 for j in keys])
                p = torch.softmax(s, 0)
                ref = sum(p[n] * v[b, h, j] for n, j in enumerate(keys))
                assert torch.allclose(out[b, h, i], ref)
    # non-causal decode form with an offset query: sees every unmasked key
    o2 = rp.attention(q[:, :, -1:], k, v, mask, causal=False)
    keys = [j for j in range(S) if mask[1, j]]
    p = torch.softmax(torch.stack([q[1, 0, -1] @ k[1, 0, j] / 8 for j in keys]), 0)
    assert torch.allclose(o2[1, 0, 0], sum(p[n] * v[1, 0, j] for n, j in enumerate(keys)))


def test_incremental_decode_equals_teacher_forced_forward():
    """Static-cache decode logits at each step == full causal forward over prompt+generated."""
    fx = load_e2e("e2e_micro")
    m = rp.OracleModel(fx.cfg, fx.weights, dtype=torch.float64)
    tr = rp.generate_output(m, fx.ids, fx.pos, fx.ex_ids, fx.mask, 6)
    S = fx.ids.shape[1]
    toks = tr.tokens
    pos = torch.cat([fx.pos, torch.stack(tr.step_positions, 1)], 1)
    full_mask = torch.cat([fx.mask, torch.ones(3, len(tr.step_positions), dtype=torch.bool)], 1)
    logits = m.forward(toks[:, :-1], pos, fx.ex_ids, full_mask, True)
    for t in range(1, len(tr.step_logits)):
        assert torch.allclose(logits[:, S + t - 1], tr.step_logits[t], atol=1e-9)


# ------------------------------------------------------------------ data format known answers
# (the reference's own tests: tests/test_data.py:97-317)

def test_data_known_answers():
    assert odf.grid_to_tokens([[1, 2, 3], [4, 5, 6]]) == [1, 2, 3, 11, 4, 5, 6, 11]
    assert odf.decode_output_grid(odf.encode_example([[1, 2], [3, 4]], [[5, 6], [7, 8]])) == \
        [[5, 6], [7, 8]]
    assert odf.decode_output_grid(odf.encode_example([[1, 2, 3]], None)) is None
    p = odf.compute_positions_3d(odf.encode_example([[1, 2, 3, 4, 5]], None))
    assert list(p[1:6, 0]) == [0, 1, 2, 3, 4]
    p = odf.compute_positions_3d(odf.encode_example([[1], [2], [3]], None))
    assert [p[1, 1], p[3, 1], p[5, 1]] == [0, 1, 2]
    toks = odf.encode_example([[1]], [[2]])
    p = odf.compute_positions_3d(toks)
    sep = toks.index(12)
    assert [p[0, 2], p[1, 2], p[sep, 2], p[sep + 1, 2], p[toks.index(13), 2]] == [0, 1, 2, 3, 4]
    sq = [[1, 2], [3, 4]]
    expect = [sq, [[3, 1], [4, 2]], [[4, 3], [2, 1]], [[2, 4], [1, 3]], [[2, 1], [4, 3]],
              [[3, 4], [1, 2]], [[1, 3], [2, 4]], [[4, 2], [3, 1]]]
    assert [f(sq) for f in odf.DIHEDRAL] == expect
