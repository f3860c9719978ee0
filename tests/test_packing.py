"""Packed prompt layout (the prefill's token list without left padding), checked on the CPU
against a per-token restatement of the padded batch it replaces."""

import numpy as np
import pytest
import torch

from mdlarc_scale_amd.engine import pack_prompt


def _brute(kv, last, B, S):
    """Tokens in row-major order of the padded batch, then the reference's lengths-1 tokens
    that fall in padding."""
    gather, row, slot = [], [], []
    head = [None] * B
    for b in range(B):
        for j in range(S):
            if j >= kv[b]:
                if b * S + j == last[b]:
                    head[b] = len(gather)
                gather.append(b * S + j)
                row.append(b)
                slot.append(j)
    n_valid = len(gather)
    for b in range(B):
        if head[b] is None:
            head[b] = len(gather)
            gather.append(last[b])
            row.append(b)
            slot.append(-1)
    return gather, row, slot, head, n_valid


@pytest.mark.parametrize("seed", range(6))
def test_pack_prompt_equals_per_token_walk(seed):
    rng = np.random.default_rng(seed)
    B, S = int(rng.integers(1, 9)), int(rng.integers(1, 40))
    kv = rng.integers(0, S + 1, size=B)
    lengths = S - kv
    # the reference's index: lengths-1 of a right-padded row, applied to the left-padded one
    last = np.arange(B) * S + np.maximum(lengths - 1, 0)
    pk = pack_prompt(kv, last, B, S, torch.device("cpu"))
    gather, row, slot, head, n_valid = _brute(kv, last, B, S)
    assert pk.n_valid == n_valid and pk.n_tokens == len(gather)
    assert pk.gather.tolist() == gather
    assert pk.token_row.tolist() == row
    assert pk.token_slot.tolist() == slot
    assert pk.head_row.tolist() == head
    offs = [sum(S - int(k) for k in kv[:b]) for b in range(B)]
    assert pk.q_offset.tolist() == offs
    # the attention kernel's packed row of query i of row b is q_offset[b] + i - kv_start[b]
    for m in range(n_valid):
        b, j = row[m], slot[m]
        assert offs[b] + j - kv[b] == m


def test_pack_prompt_rejects_foreign_last_row():
    with pytest.raises(ValueError):
        pack_prompt(np.array([0, 0]), np.array([0, 1]), 2, 4, torch.device("cpu"))
