"""Locates libhipbackend.so, the way backend-mlx's lib.ts resolves libmlxc
(packages/backend-mlx/src/lib.ts:103-141): an explicit path, then the
LAYA_HIP_PATH environment variable, then the library built in-tree next to
this package.  A missing library is an error, never a silent fallback.
"""
from __future__ import annotations

import os

LIB_NAME = "libhipbackend.so"
ENV_VAR = "LAYA_HIP_PATH"


class HipLibraryNotFound(RuntimeError):
    pass


def candidates(explicit: str | None = None) -> list[str]:
    out = []
    if explicit:
        out.append(explicit)
    env = os.environ.get(ENV_VAR)
    if env:
        out.append(os.path.join(env, LIB_NAME) if os.path.isdir(env) else env)
    out.append(os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME))
    return out


def resolve_lib(explicit: str | None = None) -> str:
    tried = candidates(explicit)
    for p in tried:
        if os.path.isfile(p):
            return p
    raise HipLibraryNotFound(
        f"{LIB_NAME} not found (tried: {', '.join(tried)}); build it with "
        f"`python -c 'import __graft_entry__ as g; g.build()'` or set {ENV_VAR}")
