"""CPU restatement of the augmentation caller of the path -- test infrastructure only.

``predict_with_augmentations`` (src/inference.py:697-760) with its batched chunk loop
(``_predict_augmentations_batched``, :763-920) and its one-prompt-at-a-time loop
(``_predict_augmentations_sequential``, :923-1003, through ``predict_grid`` :631-694), greedy
decoding only, on ``reference_path.OracleModel``.  Pinned by ``tests/golden/augment_micro.npz``,
which the reference itself wrote (tests/golden/make_golden.py): raw token streams, stop steps and
predictions per variant for chunk sizes 16 and 5, the sequential loop, constraints on and off.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import data_format as df
from . import reference_path as rp


def collect_palette(task: dict, test_idx: int, include_test_input: bool = False) -> set[int]:
    """Colours of every train input/output grid (src/inference.py:248-268)."""
    colors: set[int] = set()
    for pair in task.get("train", []):
        for key in ("input", "output"):
            g = pair.get(key)
            if g is not None:
                colors |= {int(v) for row in g for v in row}
    if include_test_input and task.get("test"):
        colors |= {int(v) for row in task["test"][test_idx]["input"] for v in row}
    return colors


def _grid_shape(grid) -> tuple[int, int] | None:
    """(h, w) of a rectangular non-empty grid, else None (src/inference.py:222-231)."""
    if not grid or not grid[0]:
        return None
    w = len(grid[0])
    return (len(grid), w) if all(len(r) == w for r in grid) else None


def infer_output_shape(task: dict) -> tuple[int, int] | None:
    """The train outputs' common shape, or None (src/inference.py:234-245)."""
    shapes = []
    for pair in task.get("train", []):
        s = _grid_shape(pair.get("output"))
        if s is None:
            return None
        shapes.append(s)
    return shapes[0] if shapes and all(s == shapes[0] for s in shapes) else None


def transform_shape(shape, dihedral_idx: int):
    """Dihedrals 1, 3, 6, 7 swap h and w (src/inference.py:271-278)."""
    if shape is None:
        return None
    return (shape[1], shape[0]) if dihedral_idx in (1, 3, 6, 7) else shape


@dataclass
class AugmentTrace:
    """What one call produced, per variant in output order."""

    predictions: list = field(default_factory=list)   # (decode(stream), dihedral, perm | None)
    generated: list = field(default_factory=list)     # generated token ids (the chunk's g_c)
    step_logits: list = field(default_factory=list)   # constrained logits [g_c, V] per variant
    raw_logits: list = field(default_factory=list)    # the same before the constraints
    prompts: list = field(default_factory=list)       # prompt tokens per variant
    widths: list = field(default_factory=list)        # padded width of each variant's chunk


def _variants(task, test_idx, use_train_examples, num_color_perms, constrain):
    """(tokens, dihedral, perm tuple, palette, shape) in the reference's order: dihedral outer,
    colour permutation inner; permutation 0 is the identity and reports None
    (src/inference.py:794-834)."""
    pairs = task["train"] if use_train_examples else []
    test_in = task["test"][test_idx]["input"]
    perms = df.color_permutations(num_color_perms, seed=42)
    base_palette = collect_palette(task, test_idx) if constrain else None
    base_shape = infer_output_shape(task) if constrain else None
    out = []
    for di, fn in enumerate(df.DIHEDRAL):
        ins = [fn(p["input"]) for p in pairs]
        outs = [fn(p["output"]) for p in pairs]
        tin = fn(test_in)
        shape = transform_shape(base_shape, di) if constrain else None
        for pi in range(num_color_perms):
            perm = perms[pi]
            palette = None
            if base_palette is not None:
                palette = {int(perm[c]) for c in base_palette} if pi > 0 else base_palette
            if pi > 0:
                cp = lambda g: [[int(perm[v]) for v in row] for row in g]   # noqa: E731
                ins_p, outs_p, tin_p = [cp(g) for g in ins], [cp(g) for g in outs], cp(tin)
            else:
                ins_p, outs_p, tin_p = ins, outs, tin
            toks: list[int] = []
            for a, b in zip(ins_p, outs_p, strict=True):
                toks += df.encode_example(a, b)
            toks += df.encode_example(tin_p, None)
            out.append((toks, di, tuple(int(v) for v in perm) if pi > 0 else None, palette,
                        shape))
    return out


def _batched_constraints(part, palette_penalty, shape_penalty):
    """Chunk constraints of the batched loop (src/inference.py:842-875): a palette row per
    prompt (all colours allowed for a prompt without one; no mask at all if no prompt has one),
    a target-shape row per prompt (-1 without one; none at all if no prompt has one)."""
    n = len(part)
    mask = torch.ones(n, 10, dtype=torch.bool)
    any_pal = False
    for i, v in enumerate(part):
        if v[3]:
            any_pal = True
            mask[i] = False
            for c in v[3]:
                if 0 <= c < 10:
                    mask[i, c] = True
    shp = torch.full((n, 2), -1, dtype=torch.long)
    any_shape = False
    for i, v in enumerate(part):
        if v[4] is not None:
            any_shape = True
            shp[i, 0], shp[i, 1] = v[4]
    return rp.OracleConstraints(palette_mask=mask if any_pal else None,
                                target_shape=shp if any_shape else None,
                                palette_penalty=palette_penalty, shape_penalty=shape_penalty)


def _sequential_constraints(v, palette_penalty, shape_penalty):
    """Constraints of one prompt in the sequential loop (src/inference.py:973-992)."""
    pal = None
    if v[3]:
        pal = torch.zeros(1, 10, dtype=torch.bool)
        for c in v[3]:
            if 0 <= c < 10:
                pal[0, c] = True
    shp = None if v[4] is None else torch.tensor([[v[4][0], v[4][1]]], dtype=torch.long)
    return rp.OracleConstraints(palette_mask=pal, target_shape=shp,
                                palette_penalty=palette_penalty, shape_penalty=shape_penalty)


def predict_with_augmentations(model: rp.OracleModel, task: dict, test_idx: int,
                               example_id: int = 0, use_train_examples: bool = True,
                               num_color_perms: int = 8, max_output_tokens: int = 900,
                               constrain_decoding: bool = False, palette_penalty: float = 2.0,
                               shape_penalty: float = 2.0, batched: bool = True,
                               max_batch_size: int = 16, decode=df.decode_output_grid
                               ) -> AugmentTrace:
    """Greedy predictions of every dihedral x colour variant of one test input.

    Batched (src/inference.py:829-918): chunks of ``max_batch_size`` prompts, each left-padded
    with END at position (0, 0, 0) to the chunk's longest prompt, one ``generate_output`` per
    chunk (so each chunk has its own ``lengths-1`` rows, budget and stop step).  Sequential
    (:953-1003): one unpadded prompt at a time without a mask (``predict_grid``).  Each row's
    prediction decodes its sequence from the last IO_SEP on (:906-913, :688-694)."""
    vs = _variants(task, test_idx, use_train_examples, num_color_perms, constrain_decoding)
    chunk = max_batch_size if batched else 1
    tr = AugmentTrace()
    for c0 in range(0, len(vs), chunk):
        part = vs[c0:c0 + chunk]
        n = len(part)
        L = max(len(v[0]) for v in part)
        ids = torch.full((n, L), df.END, dtype=torch.long)
        pos = torch.zeros(n, L, 3, dtype=torch.long)
        mask = torch.zeros(n, L, dtype=torch.bool)
        for i, v in enumerate(part):
            k = len(v[0])
            ids[i, L - k:] = torch.tensor(v[0])
            pos[i, L - k:] = torch.from_numpy(df.compute_positions_3d(v[0]))
            mask[i, L - k:] = True
        cons = None
        if constrain_decoding:
            cons = (_batched_constraints(part, palette_penalty, shape_penalty) if batched
                    else _sequential_constraints(part[0], palette_penalty, shape_penalty))
        ex = torch.full((n,), example_id, dtype=torch.long)
        g = rp.generate_output(model, ids, pos, ex, mask if batched else None, max_output_tokens,
                               True, cons)
        lg = torch.stack(g.step_logits, 1) if g.step_logits else torch.zeros(n, 0, 14)
        raw = torch.stack(g.raw_logits, 1) if g.raw_logits else torch.zeros(n, 0, 14)
        for i, v in enumerate(part):
            seq = g.tokens[i].tolist()
            seps = [j for j, t in enumerate(seq) if t == df.IO_SEP]
            tr.predictions.append((decode(seq[seps[-1]:]) if seps else None, v[1], v[2]))
            tr.generated.append(seq[L:])
            tr.step_logits.append(lg[i])
            tr.raw_logits.append(raw[i])
            tr.prompts.append(v[0])
            tr.widths.append(L)
    return tr
