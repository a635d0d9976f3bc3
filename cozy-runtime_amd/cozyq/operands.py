"""Shared activation operands: the `PreQuantized` carrier, `quantize_once` scopes, sibling
sharing and the int8 producer hook — cozyq's counterpart of cozy-runtime's
`accel/kernels.py:41-42,186-417`, with the same names, meaning and return conventions.

An encoded leaf whose GEMM takes a quantized activation asks `shared_operand` for it; leaves
reading the same input (q, k and v of one normed input, an MLP's gate and up) then quantize it
once between them. Nothing here launches a kernel: `make` callbacks do (`int8_linear.quantize`,
`fp8_linear.quantize`).
"""

from __future__ import annotations

import threading
import weakref
from collections.abc import Callable, Iterator
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass
from typing import Any

Tensor = Any

#: The providers whose leaves take a `PreQuantized` operand (`accel/kernels.py:41-42`).
ROWWISE_FP8 = "cozy.fp8-rowwise.native-leaf/1"
INT8_CONVROT = "cozy.int8-convrot256.native-leaf/1"


@dataclass(frozen=True, slots=True)
class PreQuantized:
    """An activation already in an encoded leaf's operand geometry (`accel/kernels.py:
    186-198`): `payload` `[M, K]` (int8 or E4M3), `scale` the per-row float32 scales, `shape`
    the 16-bit activation's shape (so the leaf's output reshape is unchanged) and `provider`
    the leaf family whose GEMM reads it."""

    payload: Tensor
    scale: Tensor
    shape: tuple[int, ...]
    provider: str = ROWWISE_FP8


class _Scope:
    __slots__ = ("operands", "tensor")

    def __init__(self, tensor: Tensor) -> None:
        self.tensor = tensor
        self.operands: dict[str, PreQuantized | None] = {}


_SCOPES: ContextVar[tuple[_Scope, ...]] = ContextVar("cozyq_quantize_once", default=())


@contextmanager
def quantize_once(*tensors: Tensor | None) -> Iterator[None]:
    """Inside, the encoded leaves that take one of `tensors` (that object) as input quantize it
    once between them (`accel/kernels.py:213-223`). None is skipped. A tensor must not change in
    place inside the scope."""
    added = tuple(_Scope(t) for t in tensors if t is not None)
    token = _SCOPES.set(_SCOPES.get() + added)
    try:
        yield
    finally:
        _SCOPES.reset(token)


def _geometry(x: Tensor) -> tuple[object, ...]:
    return (x.data_ptr(), tuple(x.shape), tuple(x.stride()), x.dtype)


class _Held:
    """The one operand held outside a scope for the sibling leaves that read the same unchanged
    input next (`accel/kernels.py:226-238`): its input (weakly), version, geometry and provider.
    `left` counts the reads still expected from its maker's learned group, None until learned."""

    __slots__ = ("tensor", "version", "key", "provider", "operand", "maker", "uses", "left")

    def __init__(self, x: Tensor, provider: str, operand: PreQuantized, maker: object,
                 left: int | None) -> None:  # fmt: skip
        self.tensor = weakref.ref(x, lambda _: _retire(self))
        self.version = x._version
        self.key = _geometry(x)
        self.provider = provider
        self.operand: PreQuantized | None = operand
        self.maker = maker
        self.uses = 1
        self.left = left

    def serves(self, x: Tensor, provider: str) -> bool:
        return (self.operand is not None and self.provider == provider and self.tensor() is x
                and self.version == x._version and self.key == _geometry(x))  # fmt: skip


_LOCAL = threading.local()


def _retire(held: _Held) -> None:
    """Drop the held operand now; its maker learns how many leaves read it (the most seen)."""
    if getattr(_LOCAL, "held", None) is held:
        _LOCAL.held = None
    if held.maker is not None:
        seen = getattr(held.maker, "_cozy_siblings", 1)
        held.maker._cozy_siblings = max(seen, held.uses)
    held.operand = None
    held.maker = None


def shared_operand(
    x: Tensor,
    provider: str,
    make: Callable[[], PreQuantized | None],
    consumer: object | None = None,
) -> PreQuantized | None:
    """`provider`'s operand for `x` (`accel/kernels.py:285-349`): `make()` by the first leaf to
    ask, the rest reading it — inside a `quantize_once` scope holding `x`, and otherwise for the
    sibling leaves that read one unchanged input in a row. Outside a scope one operand at most
    is held, until its maker's learned group has read it, another input is quantized, or `x`
    is freed. Without a `consumer` (a leaf recording a graph), or for an inference tensor (no
    version counter), sharing happens in scopes only. None when `make` declines."""
    for scope in _SCOPES.get():
        if scope.tensor is x:
            if provider not in scope.operands:
                scope.operands[provider] = make()
            return scope.operands[provider]
    held: _Held | None = getattr(_LOCAL, "held", None)
    if consumer is None or x.is_inference():
        if held is not None:
            _retire(held)
        return None
    if held is not None and held.serves(x, provider):
        held.uses += 1
        operand = held.operand
        if held.left is not None:
            held.left -= 1
            if held.left <= 0:
                # The group has read it: remember it, so one more reader grows the group.
                _LOCAL.last = (held.tensor, held.version, held.key, held.maker)
                _retire(held)
        return operand
    if held is not None:
        _retire(held)
    last = getattr(_LOCAL, "last", None)
    _LOCAL.last = None
    if last is not None and last[0]() is x and last[1:3] == (x._version, _geometry(x)):
        last[3]._cozy_siblings += 1
    operand = make()
    if operand is None:
        return None
    group = getattr(consumer, "_cozy_siblings", None)
    if group == 1:  # this leaf reads its input alone: nothing to hold
        return operand
    _LOCAL.held = _Held(x, provider, operand, consumer, None if group is None else group - 1)
    return operand


def int8_rows(
    x: Tensor,
    consumers: tuple[object, ...],
    *,
    norm: str | None = None,
    eps: float = 0.0,
    scale: Tensor | None = None,
    shift: Tensor | None = None,
    activation: str | None = None,
    up: Tensor | None = None,
) -> PreQuantized | None:
    """The rows a producer would hand `consumers`, `activation(norm(x)·(1 + scale) + shift)`,
    rotated and quantized for int8 in one pass (`accel/kernels.py:352-382`): the first
    consumer's `int8_prologue` decides. None unless every consumer is an encoded leaf taking
    int8.convrot's operand of x's width and the op serves this card: the caller then runs its
    own ops."""
    consumers = tuple(_baked_base(c) for c in consumers)
    if not consumers or getattr(consumers[0], "operand", None) != INT8_CONVROT:
        return None
    leader = consumers[0]
    return leader.int8_prologue(x, consumers, norm, eps, scale, shift, activation, up)


def _baked_base(module: object) -> object:
    """The leaf a composed layer hands its operand to once its update is baked into the base's
    bytes (`accel/kernels.py:385-395`)."""
    while getattr(module, "_cozy_baked", False) and not (
        getattr(module, "_forward_hooks", None) or getattr(module, "_forward_pre_hooks", None)
    ):
        base = getattr(module, "base_layer", None)
        if base is None:
            break
        module = base
    return module


def read(tensor: Any) -> Any:
    """A launch-by-pointer operand made readable (`accel/kernels.py:413-416`): a placeholder
    with a `_varena_read` binder is bound first."""
    bind = getattr(tensor, "_varena_read", None)
    return tensor if bind is None else bind()
