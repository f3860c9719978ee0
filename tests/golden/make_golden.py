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
* ``generate_color_permutations`` (src/data.py:257-278) under this container's numpy.

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

    np.savez_compressed(
        os.path.join(OUT, "color_perms.npz"),
        p8_42=rdata.generate_color_permutations(8, 42),
        p16_42=rdata.generate_color_permutations(16, 42),
        p8_7=rdata.generate_color_permutations(8, 7),
    )
    print("wrote fixtures to", OUT)


if __name__ == "__main__":
    main()
