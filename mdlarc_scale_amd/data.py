"""ARC token format, 3D positions and augmentations (input format of the inference path).

Names and semantics follow src/data.py of shyampathak22/mdlARC_scale (tokens :29-37,
encode/decode :40-117, positions :124-175, dihedral transforms :182-250, colour permutations
:257-305).  ``compute_positions_3d`` is vectorised over the token stream so that building a
B=256 batch of ~2k-token prompts stays cheap on the host.
"""

from __future__ import annotations

import numpy as np

VOCAB_SIZE = 14
START_TOKEN_ID = 10
NEWLINE_TOKEN_ID = 11
IO_SEP_TOKEN_ID = 12
END_TOKEN_ID = 13
PAD_TOKEN_ID = END_TOKEN_ID

Grid = list[list[int]]


def grid_to_tokens(grid: Grid) -> list[int]:
    """Cells row by row, each row closed by NEWLINE."""
    toks: list[int] = []
    for row in grid:
        toks.extend(int(v) for v in row)
        toks.append(NEWLINE_TOKEN_ID)
    return toks


def tokens_to_grid(tokens: list[int]) -> Grid:
    """Inverse of ``grid_to_tokens``: rows split at NEWLINE, empty rows and specials dropped."""
    rows: Grid = []
    cur: list[int] = []
    for t in tokens:
        if t == NEWLINE_TOKEN_ID:
            if cur:
                rows.append(cur)
            cur = []
        elif t < 10:
            cur.append(int(t))
    if cur:
        rows.append(cur)
    return rows


def encode_example(input_grid: Grid, output_grid: Grid | None = None) -> list[int]:
    """START input IO_SEP [output END]."""
    toks = [START_TOKEN_ID, *grid_to_tokens(input_grid), IO_SEP_TOKEN_ID]
    if output_grid is not None:
        toks += [*grid_to_tokens(output_grid), END_TOKEN_ID]
    return toks


def decode_output_grid(tokens: list[int]) -> Grid | None:
    """Grid between the first IO_SEP and the following END; None when there is none."""
    try:
        k = tokens.index(IO_SEP_TOKEN_ID)
    except ValueError:
        return None
    tail = tokens[k + 1:]
    if END_TOKEN_ID in tail:
        tail = tail[:tail.index(END_TOKEN_ID)]
    return tokens_to_grid(tail) if tail else None


def compute_positions_3d(tokens, max_x: int = 30, max_y: int = 29) -> np.ndarray:
    """(x, y, z) per token, int64 [n, 3].

    x counts colour cells since the last START / IO_SEP / NEWLINE, y counts NEWLINEs since the
    last START / IO_SEP (both clamped), z is 0 START, 1 input cell/newline, 2 IO_SEP, 3 output
    cell/newline, 4 END; END leaves the running state untouched.
    """
    t = np.asarray(tokens, dtype=np.int64).reshape(-1)
    n = t.size
    out = np.zeros((n, 3), dtype=np.int64)
    if n == 0:
        return out
    idx = np.arange(n)
    is_start, is_nl = t == START_TOKEN_ID, t == NEWLINE_TOKEN_ID
    is_sep, is_end = t == IO_SEP_TOKEN_ID, t == END_TOKEN_ID
    is_cell = ~(is_start | is_nl | is_sep | is_end)

    def since_reset(reset: np.ndarray, counted: np.ndarray) -> np.ndarray:
        # number of `counted` tokens strictly before i and after the last reset at or before i
        c = np.cumsum(counted) - counted
        last = np.maximum.accumulate(np.where(reset, idx, -1))
        base = np.where(last >= 0, np.cumsum(counted)[np.maximum(last, 0)], 0)
        return c - base

    x = since_reset(is_start | is_sep | is_nl, is_cell)
    y = since_reset(is_start | is_sep, is_nl)
    mode = np.where(is_start, 0, np.where(is_sep, 1, -1))          # last START/SEP wins
    last_mode = np.maximum.accumulate(np.where(mode >= 0, idx, -1))
    in_out = np.where(last_mode >= 0, mode[np.maximum(last_mode, 0)] == 1, False)
    z_body = np.where(in_out, 3, 1)
    out[:, 0] = np.where(is_cell, np.minimum(x, max_x), 0)
    out[:, 1] = np.where(is_cell | is_nl, np.minimum(y, max_y), 0)
    out[:, 2] = np.select([is_start, is_sep, is_end], [0, 2, 4], z_body)
    return out


# ---- dihedral group on grids (order of src/data.py:224-233) ----------------------------------
def _np(grid: Grid) -> np.ndarray:
    return np.asarray(grid, dtype=np.int64).reshape(len(grid), -1) if grid else np.zeros((0, 0))


def _ls(a: np.ndarray) -> Grid:
    return [list(map(int, r)) for r in a]


def identity(grid: Grid) -> Grid:
    return [list(r) for r in grid]


def rot90(grid: Grid) -> Grid:
    """90 degrees clockwise."""
    return _ls(np.rot90(_np(grid), k=-1))


def rot180(grid: Grid) -> Grid:
    return _ls(np.rot90(_np(grid), k=2))


def rot270(grid: Grid) -> Grid:
    """270 degrees clockwise."""
    return _ls(np.rot90(_np(grid), k=1))


def flip_h(grid: Grid) -> Grid:
    return _ls(_np(grid)[:, ::-1])


def flip_v(grid: Grid) -> Grid:
    return _ls(_np(grid)[::-1, :])


def flip_diag(grid: Grid) -> Grid:
    return _ls(_np(grid).T)


def flip_anti_diag(grid: Grid) -> Grid:
    return _ls(_np(grid).T[::-1, ::-1])


DIHEDRAL_TRANSFORMS = [identity, rot90, rot180, rot270, flip_h, flip_v, flip_diag,
                       flip_anti_diag]
_INVERSE = [0, 3, 2, 1, 4, 5, 6, 7]


def apply_dihedral_transform(input_grid: Grid, output_grid: Grid, transform_idx: int):
    f = DIHEDRAL_TRANSFORMS[transform_idx]
    return f(input_grid), f(output_grid)


def inverse_dihedral(grid: Grid, transform_idx: int) -> Grid:
    return DIHEDRAL_TRANSFORMS[_INVERSE[transform_idx]](grid)


# ---- colour permutations -----------------------------------------------------------------------
def generate_color_permutations(n_perms: int, seed: int = 42) -> np.ndarray:
    """[n_perms, 10]: colour 0 fixed, row 0 identity, later rows ``default_rng(seed)``
    permutations of 1..9 drawn in order."""
    rng = np.random.default_rng(seed)
    perms = np.tile(np.arange(10, dtype=np.int64), (n_perms, 1))
    for i in range(1, n_perms):
        perms[i, 1:] = rng.permutation(np.arange(1, 10))
    return perms


def inverse_color_perm(perm: np.ndarray) -> np.ndarray:
    inv = np.empty_like(perm)
    inv[perm] = np.arange(len(perm))
    return inv


def apply_color_perm_grid(grid: Grid, perm: np.ndarray) -> Grid:
    return _ls(np.asarray(perm)[_np(grid)]) if grid else []
