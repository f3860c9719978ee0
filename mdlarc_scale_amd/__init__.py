"""mdlarc_scale_amd -- MI355X (gfx950) HIP implementation of the TinyTransformer inference hot
path of shyampathak22/mdlARC_scale: RMSNorm, 3D RoPE, SwiGLU and static-KV-cache prefill / greedy
decode attention behind the reference's ``TinyTransformer`` / ``generate_output`` API.

The kernels live in ``libmdlarc_hip.so`` (C ABI, include/mdlarc_hip.h), built in-tree by
``python -m mdlarc_scale_amd.build``.
"""

from .checkpoint import load_model_from_checkpoint  # noqa: F401
from .data import (  # noqa: F401
    DIHEDRAL_TRANSFORMS,
    END_TOKEN_ID,
    IO_SEP_TOKEN_ID,
    NEWLINE_TOKEN_ID,
    PAD_TOKEN_ID,
    START_TOKEN_ID,
    VOCAB_SIZE,
    compute_positions_3d,
    decode_output_grid,
    encode_example,
    generate_color_permutations,
)
from .inference import (  # noqa: F401
    DecodingConstraints,
    GridStateUpdater,
    StaticKVCache,
    generate_output,
    predict_grid,
    predict_with_augmentations,
)
from .transformer import (  # noqa: F401
    TinyTransformer,
    TransformerConfig,
    create_large_model,
    create_medium_model,
    create_model,
    create_small_model,
    create_tiny_model,
)

__version__ = "0.1.0"
