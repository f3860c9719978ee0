"""Checkpoint ingest (mdlarc_scale_amd.checkpoint) against the reference's checkpoint layouts:
the training checkpoint of src/train.py:938-950 (model_state, model_config, optimizer / scheduler
state, numpy + torch RNG state, task map), the model_size-only config of src/eval.py:903-925, a
bare state dict, and safetensors.  CPU only: the files are read with weights_only=True and a
pickle that would run code is refused."""

from dataclasses import asdict

import numpy as np
import pytest
import torch

from mdlarc_scale_amd import checkpoint as C
from mdlarc_scale_amd import create_model, create_tiny_model

CALLS: list = []


def _side_effect(*args):
    CALLS.append(args)
    return args


class _Hostile:
    def __reduce__(self):
        return (_side_effect, ("payload ran",))


def _same_weights(a, b):
    sa, sb = a.state_dict(), b.state_dict()
    assert sa.keys() == sb.keys()
    for k in sa:
        assert torch.equal(sa[k], sb[k]), k


def test_reference_training_checkpoint(tmp_path):
    torch.manual_seed(0)
    m = create_tiny_model(dropout=0.0, max_seq_len=512)
    opt = torch.optim.AdamW(m.parameters(), lr=1e-3)
    m(torch.zeros(1, 4, dtype=torch.long), torch.zeros(1, 4, 3, dtype=torch.long)).sum().backward()
    opt.step()
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda s: 1.0)
    ckpt = {
        "model_state": m.state_dict(),
        "model_config": asdict(m.config),
        "optimizer_state": opt.state_dict(),
        "scheduler_state": sched.state_dict(),
        "epoch": 3,
        "global_step": 1200,
        "config": {"model_size": "tiny", "lr": 1e-3},
        "metrics": {"loss": 0.5},
        "rng_state": {"python": None, "numpy": np.random.get_state(),
                      "torch": torch.get_rng_state()},
        "task_id_to_example_id": {"abc123": 7},
    }
    path = tmp_path / "ckpt.pt"
    torch.save(ckpt, path)
    got, task_map = C.load_model_from_checkpoint(path, "cpu", return_task_id_map=True)
    assert got.config == m.config and not got.training
    _same_weights(got, m)
    assert task_map == {"abc123": 7}


def test_model_size_config_and_bare_state_dict(tmp_path):
    torch.manual_seed(1)
    tiny = create_tiny_model(dropout=0.0)
    p1 = tmp_path / "a.pt"
    torch.save({"config": {"model_size": "tiny"}, "model_state_dict": tiny.state_dict()}, p1)
    got = C.load_model_from_checkpoint(p1, "cpu")
    assert (got.config.d_model, got.config.n_layers, got.config.d_ff) == (256, 4, 704)
    _same_weights(got, tiny)
    default = create_model(dropout=0.0)
    p2 = tmp_path / "b.pt"
    torch.save(default.state_dict(), p2)
    _same_weights(C.load_model_from_checkpoint(p2, "cpu"), default)


def test_safetensors_round_trip(tmp_path):
    torch.manual_seed(2)
    m = create_model(d_model=128, n_heads=2, n_layers=2, d_ff=192, num_examples=4,
                     max_seq_len=300, dropout=0.0)
    p = tmp_path / "m.safetensors"
    C.save_safetensors(m, p)
    got = C.load_model_from_checkpoint(p, "cpu")
    assert got.config == m.config
    _same_weights(got, m)


def test_code_in_a_pickle_is_refused(tmp_path):
    p = tmp_path / "evil.pt"
    torch.save({"model_state": {}, "x": _Hostile()}, p)
    CALLS.clear()
    with pytest.raises(RuntimeError, match="weights_only"):
        C.load_model_from_checkpoint(p, "cpu")
    assert CALLS == []
