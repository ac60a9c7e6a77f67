"""retrieve_amd: an MI355X-native (gfx950) build of torchretrieve's scoring-and-selection hot
path: hand-written HIP kernels behind a C ABI (``include/retrieve_amd.h``,
``libretrieve_amd.so``), registered as the reference's ``torch.ops.retrieve.*`` /
``torch.ops.st.*`` ops.

``import retrieve_amd`` registers nothing; ``retrieve_amd.hip`` registers the
``torch.ops.retrieve.*`` ops when imported.
"""

from __future__ import annotations

import importlib

_SUBMODULES = ("hip",)


def __getattr__(name: str):
    if name in _SUBMODULES:
        return importlib.import_module(f"retrieve_amd.{name}")
    raise AttributeError(f"module 'retrieve_amd' has no attribute {name!r}")
