"""Backend registry for the Pi0 call sites (mirrors `pi0/backends/__init__.py:1-40`).

A backend is a module exposing `ALL_WRAPPERS` and `FUSED_WRAPPERS`, dicts of
call-site wrappers with identical signatures, registered in `BACKENDS`. The
TileLang backend of the reference has no gfx950 path and is not registered;
another backend can be added with `register_backend`.
"""
from __future__ import annotations

from types import SimpleNamespace

from . import hip as _hip

BACKENDS = {
    "hip": _hip,
}

DEFAULT_FUSED_OPS = tuple(sorted(_hip.FUSED_WRAPPERS))

__all__ = ["BACKENDS", "DEFAULT_FUSED_OPS", "build_table", "register_backend"]


def register_backend(name: str, module) -> None:
    if not hasattr(module, "ALL_WRAPPERS") or not hasattr(module, "FUSED_WRAPPERS"):
        raise TypeError("a backend module must define ALL_WRAPPERS and FUSED_WRAPPERS")
    BACKENDS[name] = module


def build_table(backend: str = "hip", fused: bool = True) -> SimpleNamespace:
    module = BACKENDS[backend]
    table = dict(module.ALL_WRAPPERS)
    if fused:
        table.update(module.FUSED_WRAPPERS)
    return SimpleNamespace(**table)
