"""ABI identity of the C interface in include/gsplat_hip.h.

The reference cannot call a kernel with a wrong argument list: its op schemas
are compiled into the same module as the kernels (gsplat/cuda/ext.cpp:711-808)
and bound when that module loads (gsplat/cuda/_backend.py:52-64).  Here the
library is reached through ctypes, whose argument types are written by hand
(``_lib._SIGNATURES``).  To keep the two sides from drifting apart:

- ``header_abi_hash()`` digests the header's declarations (comments and
  whitespace removed, so documentation edits do not change it);
- the build compiles that digest into the library (``gsplat_abi_version()``);
- ``_lib`` records the digest its signatures were written against and
  ``_lib.load()`` refuses a library that reports another one, before any
  entry point is bound or called;
- a CPU test checks that ``_lib``'s digest and signatures match the header.
"""

from __future__ import annotations

import hashlib
import re
from pathlib import Path
from typing import Dict, List, Tuple

HEADER = Path(__file__).resolve().parents[1] / "include" / "gsplat_hip.h"


def _code(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    return " ".join(text.split())


def header_abi_hash(path: Path = HEADER) -> str:
    """16 hex digits of SHA-256 over the header's code (no comments, single
    spaces)."""
    return hashlib.sha256(_code(Path(path).read_text()).encode()).hexdigest()[:16]


_PROTO = re.compile(r"([A-Za-z_][\w\s\*]*?)\s*\b(gsplat_\w+)\s*\(([^)]*)\)\s*;")


def _param_type(decl: str) -> str:
    """'const float *means' -> 'const float*'; 'void' -> ''."""
    decl = " ".join(decl.replace("*", " * ").split())
    if decl == "void":
        return ""
    toks = decl.split(" ")
    if len(toks) >= 2 and toks[-1] != "*" and re.fullmatch(r"[A-Za-z_]\w*", toks[-1]):
        toks = toks[:-1]  # drop the parameter name
    return " ".join(toks).replace(" *", "*")


def header_prototypes(path: Path = HEADER) -> Dict[str, Tuple[str, List[str]]]:
    """name -> (return type, parameter types) of every entry point declared
    in the header."""
    code = _code(Path(path).read_text())
    out = {}
    for ret, name, params in _PROTO.findall(code):
        ret = " ".join(ret.replace("*", " * ").split()).replace(" *", "*")
        ret = re.search(r"((?:const )?\w+\**)$", ret).group(1)
        types = [_param_type(p) for p in params.split(",")] if params.strip() else []
        out[name] = (ret, [t for t in types if t])
    return out
