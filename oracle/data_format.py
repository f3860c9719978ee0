"""Token / position / augmentation format in plain Python and numpy -- test infrastructure only.

Restates src/data.py of the reference (shyampathak22/mdlARC_scale); the product has its own
implementation in ``mdlarc_scale_amd.data`` and the tests check the two against each other and
against the reference's known answers.
"""

from __future__ import annotations

import numpy as np

START, NEWLINE, IO_SEP, END = 10, 11, 12, 13


def grid_to_tokens(grid: list[list[int]]) -> list[int]:
    """Row-major cells, NEWLINE after every row (src/data.py:40-51)."""
    out: list[int] = []
    for row in grid:
        out += list(row) + [NEWLINE]
    return out


def tokens_to_grid(tokens: list[int]) -> list[list[int]]:
    """Split on NEWLINE, drop empty rows and START/IO_SEP/END (src/data.py:54-72)."""
    grid, row = [], []
    for t in tokens:
        if t == NEWLINE:
            if row:
                grid.append(row)
                row = []
        elif t not in (START, IO_SEP, END):
            row.append(t)
    if row:
        grid.append(row)
    return grid


def encode_example(inp: list[list[int]], out: list[list[int]] | None = None) -> list[int]:
    """START in-grid IO_SEP [out-grid END] (src/data.py:75-93)."""
    toks = [START] + grid_to_tokens(inp) + [IO_SEP]
    if out is not None:
        toks += grid_to_tokens(out) + [END]
    return toks


def decode_output_grid(tokens: list[int]) -> list[list[int]] | None:
    """Cells after the first IO_SEP up to END, as a grid; None if absent (src/data.py:96-117)."""
    if IO_SEP not in tokens:
        return None
    body = []
    for t in tokens[tokens.index(IO_SEP) + 1:]:
        if t == END:
            break
        body.append(t)
    return tokens_to_grid(body) if body else None


def compute_positions_3d(tokens: list[int], max_x: int = 30, max_y: int = 29) -> np.ndarray:
    """(x, y, z) per token (src/data.py:124-175).  z: 0 START, 1 input, 2 IO_SEP, 3 output,
    4 END.  Scalar loop -- this is the small-case oracle."""
    pos = np.zeros((len(tokens), 3), dtype=np.int64)
    x = y = 0
    in_out = False
    for i, t in enumerate(tokens):
        if t == START:
            x = y = 0
            in_out = False
        elif t == NEWLINE:
            pos[i] = (0, y, 3 if in_out else 1)
            x, y = 0, min(y + 1, max_y)
        elif t == IO_SEP:
            pos[i] = (0, 0, 2)
            x = y = 0
            in_out = True
        elif t == END:
            pos[i] = (0, 0, 4)
        else:
            pos[i] = (min(x, max_x), min(y, max_y), 3 if in_out else 1)
            x += 1
    return pos


def _rot90(g):
    return [list(r) for r in zip(*g[::-1])]


def _transpose(g):
    return [list(r) for r in zip(*g)]


# src/data.py:182-233, same order: identity, rot90, rot180, rot270, flip_h, flip_v, flip_diag,
# flip_anti_diag
DIHEDRAL = [
    lambda g: [list(r) for r in g],
    _rot90,
    lambda g: [r[::-1] for r in g[::-1]],
    lambda g: _transpose(g)[::-1],
    lambda g: [r[::-1] for r in g],
    lambda g: [list(r) for r in g[::-1]],
    _transpose,
    lambda g: [r[::-1] for r in _transpose(g)[::-1]],
]


def color_permutations(n: int, seed: int = 42) -> np.ndarray:
    """[n, 10] colour maps: 0 fixed, row 0 identity, rows 1.. a numpy ``default_rng(seed)``
    permutation of 1..9 each (src/data.py:257-278)."""
    rng = np.random.default_rng(seed)
    perms = np.zeros((n, 10), dtype=np.int64)
    perms[0, 1:] = np.arange(1, 10)
    for i in range(1, n):
        perms[i, 1:] = rng.permutation(np.arange(1, 10))
    return perms
