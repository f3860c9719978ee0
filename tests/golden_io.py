"""Load the golden fixtures written by tests/golden/make_golden.py."""

from __future__ import annotations

import os
from dataclasses import dataclass

import numpy as np
import torch

from oracle.reference_path import OracleConfig

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@dataclass
class E2EFixture:
    cfg: OracleConfig
    weights: dict[str, torch.Tensor]
    ids: torch.Tensor
    pos: torch.Tensor
    mask: torch.Tensor
    ex_ids: torch.Tensor
    max_new: int
    fwd_logits: torch.Tensor
    gen: torch.Tensor
    step_logits: torch.Tensor
    step_pos: torch.Tensor
    single_prompt: torch.Tensor
    single_gen: torch.Tensor


def load_e2e(name: str) -> E2EFixture:
    """Fixture ``name``; the stop variant shares the base fixture's weights except lm_head."""
    base = np.load(os.path.join(GOLDEN, "e2e_micro.npz"))
    f = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    w = {k[2:]: torch.from_numpy(base[k]) for k in base.files if k.startswith("w:")}
    w.update({k[2:]: torch.from_numpy(f[k]) for k in f.files if k.startswith("w:")})
    d, h, nl, ff, nex, msl = f["cfg"].tolist()
    t = lambda k: torch.from_numpy(f[k])  # noqa: E731
    return E2EFixture(OracleConfig(d, h, nl, ff, nex, msl), w, t("ids"), t("pos"), t("mask"),
                      t("ex_ids"), int(f["max_new"]), t("fwd_logits"), t("gen"), t("step_logits"),
                      t("step_pos"), t("single_prompt"), t("single_gen"))


def constraint_cases() -> list[dict]:
    """Cases of tests/golden/constraints.npz: inputs of the reference's _apply_logit_constraints
    (logits [B, V], grid state, optional palette / target shape, penalties, disallowed tokens)
    and its output."""
    f = np.load(os.path.join(GOLDEN, "constraints.npz"))
    out = []
    for i in range(int(f["n_cases"])):
        k = f"c{i}_"
        g = lambda n: torch.from_numpy(f[k + n]) if k + n in f.files else None  # noqa: E731
        pp, sp = f[k + "penalties"].tolist()
        out.append(dict(logits=g("logits")[:, 0], gx=g("gx"), gy=g("gy"), palette=g("palette"),
                        shape=g("shape"), palette_penalty=pp, shape_penalty=sp,
                        disallow=tuple(f[k + "disallow"].tolist()), out=g("out")[:, 0]))
    return out


@dataclass
class AugmentRun:
    stop_model: bool
    batched: bool
    chunk: int
    constrain: bool
    streams: list[tuple[int, ...]]      # per variant: the tokens its prediction is decoded from
    gen: list[list[int]]                # per variant: the generated tokens (its chunk's g_c)
    gaps: list[np.ndarray]              # per variant: top-2 gap of the constrained logits per step
    aug: list[tuple[int, tuple | None]]  # per variant: (dihedral, colour permutation | None)


@dataclass
class AugmentFixture:
    task: dict
    num_color_perms: int
    max_new: int
    example_id: int
    runs: list[AugmentRun]
    grids: list                         # decoded predictions of the default call (stop model)


def load_augment() -> AugmentFixture:
    """tests/golden/augment_micro.npz: the reference's predict_with_augmentations runs."""
    import json

    f = np.load(os.path.join(GOLDEN, "augment_micro.npz"))
    runs = []
    for r in range(int(f["n_runs"])):
        k = f"r{r}_"
        stop, batched, chunk, constrain = f[k + "run"].tolist()
        streams = [tuple(int(t) for t in row if t >= 0) for row in f[k + "streams"]]
        gen = [[int(t) for t in row if t >= 0] for row in f[k + "gen"]]
        gaps = [row[~np.isnan(row)] for row in f[k + "gaps"]]
        aug = [(int(a[0]), None if a[1] < 0 else tuple(int(v) for v in a[1:]))
               for a in f[k + "aug"]]
        runs.append(AugmentRun(bool(stop), bool(batched), int(chunk), bool(constrain), streams,
                               gen, gaps, aug))
    perms, max_new, ex = f["params"].tolist()
    return AugmentFixture(json.loads(str(f["task"])), perms, max_new, ex, runs,
                          json.loads(str(f["grids_json"])))


def augment_weights(stop_model: bool) -> tuple[OracleConfig, dict[str, torch.Tensor]]:
    """The micro model of the augmentation fixture: the e2e fixture weights (the stop variant's
    lm_head for the stop model) rounded to bf16 once."""
    fx = load_e2e("e2e_micro_stop" if stop_model else "e2e_micro")
    return fx.cfg, {k: v.to(torch.bfloat16).float() for k, v in fx.weights.items()}
