"""Write the golden input/output vectors that pin the CPU oracle's end-to-end behaviour.

This script runs ONLY in the build container, where the reference checkout is mounted at
/root/reference.  It imports the reference's own Python (never copies it) and records the
outputs of the functions whose behaviour no closed form pins:

* ``generate_output`` (src/inference.py:487-628) on a left-padded, variable-length batch, including
  the ``lengths-1`` last-token index used by ``_prefill`` (src/inference.py:420-424) and
  ``_derive_initial_state_from_prompt`` (src/inference.py:171-221), per-step logits and the
  grid-state positions fed to every decode step (``GridStateUpdater.update``,
  src/inference.py:127-168), and the stop-on-END break (src/inference.py:589-595);
* ``TinyTransformer.forward`` (src/transformer.py:562-599) logits on the same padded batch;
* ``GridStateUpdater`` traces and ``_derive_initial_state_from_prompt`` on ragged masks;
* ``generate_color_permutations`` (src/data.py:257-278) under this container's numpy;
* ``_apply_logit_constraints`` (src/inference.py:285-364) on random logits, grid states, palettes
  and target shapes covering every branch (broadcast rows, mismatched batches, rows without a
  shape, boundary x == w / y == h) -> ``constraints.npz``;
* ``predict_with_augmentations`` (src/inference.py:697-1003) on a small task with the micro model
  (weights rounded to bf16 so a bf16-weight GPU path runs the very same weights): the batched
  chunk loop at chunk sizes 16 and 5 and the sequential loop, constraints on and off, recording
  per variant the raw token stream the prediction is decoded from, the generated tokens and the
  top-2 gap of the constrained logits at every step -> ``augment_micro.npz``.

Weights are NOT the reference's random init: they are drawn here from a seeded numpy generator
(perturbed norm gains and biases, so those code paths are exercised) and loaded into the
reference model with ``load_state_dict``; the same arrays are stored in the fixture so the oracle
runs on identical weights.

Run:  python tests/golden/make_golden.py      (writes tests/golden/*.npz)
"""

from __future__ import annotations

import os
import sys

import numpy as np

REF = "/root/reference"
OUT = os.path.dirname(os.path.abspath(__file__))

D_MODEL, N_HEADS, N_LAYERS, D_FF, N_EX, MAX_SEQ = 128, 2, 2, 192, 4, 160


def _weights(rng: np.random.Generator, end_boost: float) -> dict[str, np.ndarray]:
    d, f = D_MODEL, D_FF
    w: dict[str, np.ndarray] = {}

    def lin(o: int, i: int) -> np.ndarray:
        a = np.sqrt(6.0 / (i + o))
        return rng.uniform(-a, a, size=(o, i)).astype(np.float32)

    w["token_embed.weight"] = rng.normal(0, 0.5, size=(14, d)).astype(np.float32)
    w["example_embed.weight"] = rng.normal(0, 0.5, size=(N_EX, d)).astype(np.float32)
    for i in range(N_LAYERS):
        p = f"blocks.{i}."
        w[p + "ln1.weight"] = (1 + 0.1 * rng.normal(size=d)).astype(np.float32)
        w[p + "attn.qkv_proj.weight"] = lin(3 * d, d)
        w[p + "attn.out_proj.weight"] = lin(d, d)
        w[p + "ln2.weight"] = (1 + 0.1 * rng.normal(size=d)).astype(np.float32)
        w[p + "ffn.fc_gate.weight"] = lin(f, d)
        w[p + "ffn.fc_gate.bias"] = (0.02 * rng.normal(size=f)).astype(np.float32)
        w[p + "ffn.fc_up.weight"] = lin(f, d)
        w[p + "ffn.fc_up.bias"] = (0.02 * rng.normal(size=f)).astype(np.float32)
        w[p + "ffn.fc_down.weight"] = lin(d, f)
        w[p + "ffn.fc_down.bias"] = (0.02 * rng.normal(size=d)).astype(np.float32)
    w["ln_f.weight"] = (1 + 0.1 * rng.normal(size=d)).astype(np.float32)
    head = lin(14, d) * 4.0
    head[13] *= end_boost
    w["lm_head.weight"] = head.astype(np.float32)
    return w


def _grid(rng: np.random.Generator, h: int, w: int) -> list[list[int]]:
    g = rng.integers(1, 10, size=(h, w))
    g[rng.random((h, w)) < 0.5] = 0
    return g.tolist()


def main() -> None:
    sys.path.insert(0, REF)
    import torch

    from src import data as rdata
    from src import inference as rinf
    from src.transformer import TransformerConfig, TinyTransformer

    torch.manual_seed(0)
    rng = np.random.default_rng(20261201)

    # ---------------- prompts: left-padded, variable length ----------------
    specs = [  # (pairs of (in_h,in_w,out_h,out_w)), test (h,w)
        ([(2, 3, 2, 3)], (2, 2)),                        # short: quirk index falls in the pad
        ([(3, 4, 3, 4), (2, 2, 2, 2)], (3, 3)),          # medium: quirk index mid-prompt
        ([(4, 5, 4, 5), (3, 3, 3, 3)], (4, 4)),          # longest: no padding
    ]
    prompts = []
    for pairs, (th, tw) in specs:
        toks: list[int] = []
        for ih, iw, oh, ow in pairs:
            toks += rdata.encode_example(_grid(rng, ih, iw), _grid(rng, oh, ow))
        toks += rdata.encode_example(_grid(rng, th, tw), None)
        prompts.append(toks)
    S = max(len(p) for p in prompts)
    B = len(prompts)
    ids = np.full((B, S), rdata.END_TOKEN_ID, dtype=np.int64)
    pos = np.zeros((B, S, 3), dtype=np.int64)
    mask = np.zeros((B, S), dtype=bool)
    for b, p in enumerate(prompts):
        n = len(p)
        ids[b, S - n:] = p
        pos[b, S - n:] = rdata.compute_positions_3d(p)
        mask[b, S - n:] = True
    ex_ids = np.array([1, 2, 3], dtype=np.int64)

    cfg = TransformerConfig(d_model=D_MODEL, n_heads=N_HEADS, n_layers=N_LAYERS, d_ff=D_FF,
                            num_examples=N_EX, max_seq_len=MAX_SEQ, dropout=0.0)

    fixtures = {}
    for name, end_boost, max_new in (("e2e_micro", 1.0, 24), ("e2e_micro_stop", 2.2, 40)):
        w = _weights(np.random.default_rng(7), end_boost)
        model = TinyTransformer(cfg)
        model.load_state_dict({k: torch.from_numpy(v) for k, v in w.items()}, strict=True)
        model.eval()

        t_ids, t_pos = torch.from_numpy(ids), torch.from_numpy(pos)
        t_mask, t_ex = torch.from_numpy(mask), torch.from_numpy(ex_ids)
        with torch.no_grad():
            fwd = model(t_ids, t_pos, t_ex, attention_mask=t_mask, is_causal=True).numpy()

        rec_logits: list[np.ndarray] = []
        rec_pos: list[np.ndarray] = []
        orig_prefill, orig_decode = rinf._prefill, rinf._decode_step

        def prefill_rec(*a, **k):
            out = orig_prefill(*a, **k)
            rec_logits.append(out[:, 0].detach().numpy().copy())
            return out

        def decode_rec(model_, token, position, *a, **k):
            rec_pos.append(position[:, 0].detach().numpy().copy())
            out = orig_decode(model_, token, position, *a, **k)
            rec_logits.append(out[:, 0].detach().numpy().copy())
            return out

        rinf._prefill, rinf._decode_step = prefill_rec, decode_rec
        try:
            with torch.no_grad():
                gen = rinf.generate_output(model, t_ids, t_pos, t_ex, attention_mask=t_mask,
                                           max_new_tokens=max_new, temperature=0.0).numpy()
        finally:
            rinf._prefill, rinf._decode_step = orig_prefill, orig_decode

        # single row, no mask, no example ids (defaults path: example_ids -> zeros)
        p0 = prompts[1]
        with torch.no_grad():
            gen1 = rinf.generate_output(model, torch.tensor([p0]),
                                        torch.from_numpy(rdata.compute_positions_3d(p0)[None]),
                                        max_new_tokens=12).numpy()

        # the stop variant differs from the base weights only in lm_head; store just that
        keep = w if name == "e2e_micro" else {"lm_head.weight": w["lm_head.weight"]}
        fixtures[name] = dict(
            **{"w:" + k: v for k, v in keep.items()},
            cfg=np.array([D_MODEL, N_HEADS, N_LAYERS, D_FF, N_EX, MAX_SEQ], dtype=np.int64),
            ids=ids, pos=pos, mask=mask, ex_ids=ex_ids, max_new=np.int64(max_new),
            fwd_logits=fwd, gen=gen, step_logits=np.stack(rec_logits, 1),
            step_pos=np.stack(rec_pos, 1) if rec_pos else np.zeros((B, 0, 3), np.int64),
            single_prompt=np.array(p0, dtype=np.int64), single_gen=gen1,
        )
        print(name, "S", S, "gen", gen.shape, "steps", len(rec_logits),
              "last tokens", gen[:, S:].tolist())

    for name, arrs in fixtures.items():
        np.savez_compressed(os.path.join(OUT, f"{name}.npz"), **arrs)

    # ---------------- grid-state traces ----------------
    grng = np.random.default_rng(99)
    n_rows, n_steps = 16, 200
    toks = grng.choice(14, size=(n_rows, n_steps), p=[0.045] * 10 + [0.05, 0.3, 0.1, 0.1])
    toks = toks.astype(np.int64)
    x0 = grng.integers(0, 35, size=n_rows)
    y0 = grng.integers(0, 33, size=n_rows)
    io0 = grng.random(n_rows) < 0.5
    upd = rinf.GridStateUpdater(n_rows, torch.device("cpu"))
    upd.set_state(torch.from_numpy(x0), torch.from_numpy(y0), torch.from_numpy(io0))
    trace = []
    for s in range(n_steps):
        trace.append(upd.update(torch.from_numpy(toks[:, s])).numpy().copy())
    final = np.stack([upd.x.numpy(), upd.y.numpy(), upd.in_output.numpy().astype(np.int64)], 1)

    # initial state derivation on ragged masks (left pad, right pad, holes, empty rows)
    L = 40
    p_ids = grng.integers(0, 14, size=(12, L)).astype(np.int64)
    p_pos = np.stack([grng.integers(0, 33, size=(12, L)), grng.integers(0, 33, size=(12, L)),
                      grng.integers(0, 5, size=(12, L))], -1).astype(np.int64)
    p_mask = np.zeros((12, L), dtype=bool)
    for r in range(12):
        kind = r % 4
        n = int(grng.integers(0, L + 1))
        if kind == 0:
            p_mask[r, L - n:] = True
        elif kind == 1:
            p_mask[r, :n] = True
        elif kind == 2:
            p_mask[r] = grng.random(L) < 0.6
        # kind 3: all False
    ix, iy, iio = rinf._derive_initial_state_from_prompt(
        torch.from_numpy(p_ids), torch.from_numpy(p_pos), torch.from_numpy(p_mask), 30, 29)
    np.savez_compressed(
        os.path.join(OUT, "grid_state.npz"),
        tokens=toks, x0=x0, y0=y0, io0=io0, positions=np.stack(trace, 1), final=final,
        p_ids=p_ids, p_pos=p_pos, p_mask=p_mask,
        init=np.stack([ix.numpy(), iy.numpy(), iio.numpy().astype(np.int64)], 1),
    )

    _constraint_cases(rinf)
    _augment_runs(rinf, cfg, TinyTransformer)

    np.savez_compressed(
        os.path.join(OUT, "color_perms.npz"),
        p8_42=rdata.generate_color_permutations(8, 42),
        p16_42=rdata.generate_color_permutations(16, 42),
        p8_7=rdata.generate_color_permutations(8, 7),
    )
    print("wrote fixtures to", OUT)


def _constraint_cases(rinf) -> None:
    """Inputs and outputs of the reference's ``_apply_logit_constraints``."""
    import torch

    crng = np.random.default_rng(4242)
    cases = []

    def add(B, pal, shape, pp, sp, disallow=(10, 12), grid_b=None, x=None, y=None):
        gb = B if grid_b is None else grid_b
        lg = (3.0 * crng.standard_normal((B, 1, 14))).astype(np.float32)
        gx = crng.integers(0, 31, size=gb) if x is None else np.asarray(x)
        gy = crng.integers(0, 30, size=gb) if y is None else np.asarray(y)
        cases.append(dict(B=B, logits=lg, gx=gx.astype(np.int64), gy=gy.astype(np.int64),
                          pal=pal, shape=shape, pp=pp, sp=sp, disallow=tuple(disallow)))

    B = 12
    pal = crng.random((B, 10)) < 0.6
    pal[3] = True                                            # a row with every colour allowed
    shp = np.stack([crng.integers(1, 31, B), crng.integers(1, 31, B)], 1)
    shp[[2, 7]] = -1                                         # rows without a target shape
    shp[5, 0] = -1                                           # h < 0 alone also means "no shape"
    x = crng.integers(0, 31, B)
    y = crng.integers(0, 30, B)
    x[0], y[0] = shp[0, 1], shp[0, 0]                        # boundary: x == w, y == h
    x[1], y[1] = shp[1, 1] - 1, shp[1, 0] - 1                # just inside
    add(B, pal, shp, 2.0, 2.0, x=x, y=y)
    add(8, crng.random((1, 10)) < 0.5, np.array([[4, 6]]), 0.5, 3.25)          # 1-row broadcast
    add(6, crng.random((3, 10)) < 0.5, None, 2.0, 2.0, disallow=(13,))         # mismatch: skip
    add(6, None, np.stack([crng.integers(1, 9, 4), crng.integers(1, 9, 4)], 1), 2.0, 2.0)
    add(5, None, np.full((5, 2), -1), 2.0, 2.0)                                 # no shape at all
    add(4, np.ones((4, 10), bool), np.array([[3, 3]]), 1.0, 7.5, grid_b=1)      # early return
    add(4, crng.random((4, 10)) < 0.5, np.array([[2, 9], [9, 2], [5, 5], [1, 1]]), 2.0, 2.0,
        disallow=())
    add(16, crng.random((16, 10)) < 0.3, np.stack([crng.integers(0, 31, 16),
                                                    crng.integers(0, 31, 16)], 1), 2.0, 2.0)
    add(3, np.zeros((3, 10), bool), None, 1e4, 2.0)                             # huge penalty

    out = {}
    for i, c in enumerate(cases):
        upd = rinf.GridStateUpdater(len(c["gx"]), torch.device("cpu"))
        upd.set_state(torch.from_numpy(c["gx"]), torch.from_numpy(c["gy"]),
                      torch.zeros(len(c["gx"]), dtype=torch.bool))
        cons = rinf.DecodingConstraints(
            palette_mask=None if c["pal"] is None else torch.from_numpy(np.asarray(c["pal"])),
            target_shape=None if c["shape"] is None else torch.from_numpy(
                np.asarray(c["shape"], dtype=np.int64)),
            palette_penalty=c["pp"], shape_penalty=c["sp"], disallow_tokens=c["disallow"])
        res = rinf._apply_logit_constraints(torch.from_numpy(c["logits"].copy()), upd, cons)
        k = f"c{i}_"
        out[k + "logits"] = c["logits"]
        out[k + "gx"], out[k + "gy"] = c["gx"], c["gy"]
        if c["pal"] is not None:
            out[k + "palette"] = np.asarray(c["pal"], dtype=bool)
        if c["shape"] is not None:
            out[k + "shape"] = np.asarray(c["shape"], dtype=np.int64)
        out[k + "penalties"] = np.array([c["pp"], c["sp"]], dtype=np.float32)
        out[k + "disallow"] = np.array(c["disallow"], dtype=np.int64)
        out[k + "out"] = res.numpy()
    out["n_cases"] = np.int64(len(cases))
    np.savez_compressed(os.path.join(OUT, "constraints.npz"), **out)
    print("constraints:", len(cases), "cases")


AUG_TASK = {"train": [{"input": [[1, 2, 3, 4, 5, 6]], "output": [[6], [5], [4], [3], [2], [1]]},
                      {"input": [[7, 0], [0, 7]], "output": [[0, 7], [7, 0]]}],
            "test": [{"input": [[1, 0, 2, 0, 3]]}]}
# (model, batched, max_batch_size, constrain_decoding); "stop" ends rows at many different steps,
# "open" rarely emits END and runs into the max_seq_len budgets
AUG_RUNS = [("stop", True, 16, False), ("stop", True, 5, False), ("stop", False, 1, False),
            ("stop", True, 5, True), ("stop", False, 1, True), ("open", True, 16, False),
            ("open", False, 1, True)]
AUG_PERMS, AUG_MAX_NEW, AUG_EXAMPLE = 3, 130, 1


def _augment_runs(rinf, cfg, TinyTransformer) -> None:
    """Raw per-variant outputs of the reference's augmentation caller."""
    import json

    import torch

    models = {}
    for name, boost in (("stop", 2.2), ("open", 1.0)):
        w = _weights(np.random.default_rng(7), boost)
        m = TinyTransformer(cfg)
        m.load_state_dict({k: torch.from_numpy(v).to(torch.bfloat16).float()
                           for k, v in w.items()}, strict=True)
        models[name] = m.eval()

    out = {"task": np.array(json.dumps(AUG_TASK)),
           "params": np.array([AUG_PERMS, AUG_MAX_NEW, AUG_EXAMPLE], dtype=np.int64),
           "end_boost": np.array([2.2, 1.0], dtype=np.float64)}
    orig_gen, orig_cons, orig_dec = (rinf.generate_output, rinf._apply_logit_constraints,
                                     rinf.decode_output_grid)
    for r, (mname, batched, chunk, constrain) in enumerate(AUG_RUNS):
        calls, logs = [], []

        def cons_rec(logits, grid_state, constraints):
            res = orig_cons(logits, grid_state, constraints)
            logs.append(res[:, 0].detach().clone())
            return res

        def gen_rec(model, input_ids, *a, **k):
            start = len(logs)
            res = orig_gen(model, input_ids, *a, **k)
            calls.append((input_ids.shape[1], res.detach().clone(),
                          torch.stack(logs[start:], 1) if len(logs) > start else None))
            return res

        rinf.generate_output, rinf._apply_logit_constraints = gen_rec, cons_rec
        rinf.decode_output_grid = lambda toks: tuple(toks)
        try:
            with torch.no_grad():
                if batched:
                    base_palette = rinf._collect_palette(AUG_TASK, 0) if constrain else None
                    base_shape = rinf._infer_output_shape(AUG_TASK) if constrain else None
                    preds = rinf._predict_augmentations_batched(
                        models[mname], AUG_TASK, 0, torch.device("cpu"), AUG_EXAMPLE, True,
                        AUG_PERMS, AUG_MAX_NEW, 1, 0.0, None, constrain, base_palette,
                        base_shape, 2.0, 2.0, False, max_batch_size=chunk)
                else:
                    preds = rinf.predict_with_augmentations(
                        models[mname], AUG_TASK, 0, torch.device("cpu"), example_id=AUG_EXAMPLE,
                        num_color_perms=AUG_PERMS, max_output_tokens=AUG_MAX_NEW,
                        constrain_decoding=constrain, batched=False)
        finally:
            rinf.generate_output, rinf._apply_logit_constraints = orig_gen, orig_cons
            rinf.decode_output_grid = orig_dec
        gens, gaps = [], []
        for L, res, lg in calls:
            for i in range(res.shape[0]):
                gens.append(res[i, L:].tolist())
                top = lg[i].topk(2, dim=-1).values
                gaps.append((top[:, 0] - top[:, 1]).tolist())
        n, gmax = len(preds), max(len(g) for g in gens)
        smax = max(len(p[0]) for p in preds)
        streams = np.full((n, smax), -1, dtype=np.int64)
        genarr = np.full((n, gmax), -1, dtype=np.int64)
        gaparr = np.full((n, gmax), np.nan, dtype=np.float32)
        for i, (p, g, gp) in enumerate(zip(preds, gens, gaps)):
            streams[i, :len(p[0])] = p[0]
            genarr[i, :len(g)] = g
            gaparr[i, :len(gp)] = gp
        k = f"r{r}_"
        out[k + "run"] = np.array([mname == "stop", batched, chunk, constrain], dtype=np.int64)
        out[k + "streams"], out[k + "gen"], out[k + "gaps"] = streams, genarr, gaparr
        out[k + "aug"] = np.array([[p[1]] + (list(p[2]) if p[2] else [-1] * 10) for p in preds],
                                  dtype=np.int64)
        print(f"augment run {r} {AUG_RUNS[r]}: {n} variants, "
              f"{len({len(g) for g in gens})} distinct generated lengths, "
              f"min top-2 gap {np.nanmin(gaparr):.4f}")
    # one run decoded to grids by the reference's own decode_output_grid
    with torch.no_grad():
        preds = rinf.predict_with_augmentations(
            models["stop"], AUG_TASK, 0, torch.device("cpu"), example_id=AUG_EXAMPLE,
            num_color_perms=AUG_PERMS, max_output_tokens=AUG_MAX_NEW)
    out["grids_json"] = np.array(json.dumps([p[0] for p in preds]))
    out["n_runs"] = np.int64(len(AUG_RUNS))
    np.savez_compressed(os.path.join(OUT, "augment_micro.npz"), **out)


if __name__ == "__main__":
    main()
