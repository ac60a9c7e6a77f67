"""Builds ``oracle/_ref/libsilvertorch_cpu_ref.so``: the reference's own CPU ops (Meta's
SilverTorch C++ as vendored in rmnigm/retrieve), compiled with g++ from the source files where
they lie under ``/root/reference`` -- nothing is copied -- against the libtorch this image's
torch ships. TEST INFRASTRUCTURE: only ``tests/golden/make_ref_fixtures.py`` loads the library,
in this container, to write fixtures; nothing on the product path or the GPU box uses it.

The sources (``silvertorch/silvertorch/ops/csrc``): ``bloom_indexer.cpp`` (the CPU Bloom build),
``bloom_index_util.cpp`` (the plan encoding), ``expression_query_parser.cpp`` (the expression
parser), ``bloom_index_search.cpp`` (the CPU Bloom search, full and partial) and
``fused_kmean_ann.cpp`` (the CPU scorer). They register ``torch.ops.st.*`` CPU kernels when
loaded with ``torch.ops.load_library``; the CUDA sources need nvcc and are not built.

Usage: ``python oracle/build_ref.py`` (does nothing, successfully, when ``/root/reference`` is
absent)."""

from __future__ import annotations

import os
import subprocess
import sys

REF = os.environ.get("RETRIEVE_REFERENCE", "/root/reference")
CSRC = os.path.join(REF, "silvertorch", "silvertorch", "ops", "csrc")
SOURCES = ("bloom_indexer.cpp", "bloom_index_util.cpp", "expression_query_parser.cpp",
           "bloom_index_search.cpp", "fused_kmean_ann.cpp")
HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_ref")
OUT = os.path.join(OUT_DIR, "libsilvertorch_cpu_ref.so")


def build(jobs: int = 5) -> str | None:
    """Compiles the sources (in parallel) and links the library; returns its path, or None when
    the reference checkout is absent."""
    if not os.path.isdir(CSRC):
        return None
    import torch
    from torch.utils import cpp_extension

    os.makedirs(OUT_DIR, exist_ok=True)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    flags = ["-O2", "-std=c++17", "-fPIC", "-w", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
             f"-I{CSRC}"] + [f"-I{p}" for p in cpp_extension.include_paths()]
    objs = []
    procs = []
    for src in SOURCES:
        obj = os.path.join(OUT_DIR, src.replace(".cpp", ".o"))
        objs.append(obj)
        procs.append(subprocess.Popen(["g++", *flags, "-c", os.path.join(CSRC, src), "-o", obj]))
        if len(procs) >= jobs:
            if procs.pop(0).wait() != 0:
                raise RuntimeError("compiling the reference's CPU ops failed")
    for p in procs:
        if p.wait() != 0:
            raise RuntimeError("compiling the reference's CPU ops failed")
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    subprocess.run(["g++", "-shared", "-o", OUT, *objs, f"-L{libdir}", "-ltorch", "-ltorch_cpu",
                    "-lc10", f"-Wl,-rpath,{libdir}"], check=True)
    for obj in objs:
        os.remove(obj)
    return OUT


if __name__ == "__main__":
    path = build()
    print(path or f"{CSRC} not found: nothing built", file=sys.stderr)
