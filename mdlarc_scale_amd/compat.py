"""Module aliases that put this package under the reference's import names.

shyampathak22/mdlARC_scale imports the model and the inference engine as ``src.transformer`` and
``src.inference`` (src/eval.py:22-31, src/train.py:38-44, its tests).  ``install()`` registers
this package's modules under those names inside the reference's own ``src`` package, so
``src.eval`` / ``src.voting`` / ``src.train`` run unchanged on the HIP path:

    import mdlarc_scale_amd.compat as compat
    compat.install()                 # before anything imports src.eval / src.train
    from src.eval import main        # the reference's evaluation, now on the MI355X kernels

``src.data`` stays the reference's own module (its dataset / download code is used by train and
eval); this package's inference path uses its own copy of the token format.
"""

from __future__ import annotations

import importlib
import sys

ALIASED = ("transformer", "inference")


def install(package: str = "src") -> None:
    """Alias ``<package>.transformer`` and ``<package>.inference`` to this package's modules.
    Raises ``RuntimeError`` if either was already imported from the reference (the aliases
    must be in place before the first import, or two model classes would coexist)."""
    from . import inference, transformer

    mods = {"transformer": transformer, "inference": inference}
    pkg = importlib.import_module(package)
    for name in ALIASED:
        full = f"{package}.{name}"
        prev = sys.modules.get(full)
        if prev is not None and prev is not mods[name]:
            raise RuntimeError(f"{full} was imported before compat.install(); call install() "
                               "first")
        sys.modules[full] = mods[name]
        setattr(pkg, name, mods[name])


def installed(package: str = "src") -> bool:
    from . import inference, transformer

    return (sys.modules.get(f"{package}.transformer") is transformer and
            sys.modules.get(f"{package}.inference") is inference)
