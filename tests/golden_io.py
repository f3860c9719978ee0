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
