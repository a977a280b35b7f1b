"""The operation table the decoder pipeline is written against (mirrors `pi0/ops.py:21-52`).

`op_table(fused, backend, plan)` resolves every call-site name to one wrapper
before capture; `plan` maps individual op names to a backend. Unlike the
reference, an op that the chosen backend cannot provide raises here instead
of being silently dropped from the table.
"""
from __future__ import annotations

from types import SimpleNamespace

from .backends import BACKENDS, build_table as _build_table


def op_table(fused: bool = True, backend: str = "hip",
             plan: dict[str, str] | None = None) -> SimpleNamespace:
    if backend not in BACKENDS:
        raise KeyError(f"unknown backend {backend!r}; registered: {sorted(BACKENDS)}")
    if plan is None:
        return _build_table(backend, fused=fused)
    unknown = set(plan) - set(_op_names(backend))
    if unknown:
        raise KeyError(f"plan names ops the {backend!r} backend does not have: {sorted(unknown)}")
    table = {}
    for op_name in _op_names(backend):
        chosen = plan.get(op_name, backend)
        if chosen not in BACKENDS:
            raise KeyError(f"unknown backend {chosen!r} for {op_name}")
        module = BACKENDS[chosen]
        if fused and op_name in module.FUSED_WRAPPERS:
            table[op_name] = module.FUSED_WRAPPERS[op_name]
        elif op_name in module.ALL_WRAPPERS:
            table[op_name] = module.ALL_WRAPPERS[op_name]
        else:
            raise KeyError(f"backend {chosen!r} does not implement {op_name}")
    return SimpleNamespace(**table)


def _op_names(backend: str) -> list[str]:
    module = BACKENDS[backend]
    return sorted(set(module.ALL_WRAPPERS) | set(module.FUSED_WRAPPERS))


def op_names(fused: bool = True, backend: str = "hip") -> list[str]:
    return sorted(vars(op_table(fused, backend=backend)))
