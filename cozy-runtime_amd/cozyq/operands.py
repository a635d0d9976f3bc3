"""Activation operands shared between encoded leaves, and the int8 producer hand-off.

The public names and their meaning are those of cozy-runtime's operand API
(`src/cozy_runtime/accel/kernels.py:41-42,186-198,212-222,285-416`): `PreQuantized`,
`quantize_once`, `shared_operand`, `int8_rows`, `read` and the two operand provider names. The
sharing rules S1–S5 are implemented by `_Sharing`, a per-thread state machine:
- S1: `quantize_once` scopes memoize one operand per (tensor, provider).
- S2: there is no sharing without a consumer or for inference tensors.
- S3: one operand is held per thread, keyed by the input's identity, version and geometry.
- S4: reader groups are learned per maker.
- S5: the held operand is dropped on another ask or on the input's death.
Nothing here launches a kernel: the `make` callbacks do.
"""

from __future__ import annotations

import threading
import weakref
from collections.abc import Callable, Iterator
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass, field
from typing import Any

Tensor = Any
Make = Callable[[], "PreQuantized | None"]

#: Operand geometries a leaf's GEMM reads (`accel/kernels.py:41-42`).
ROWWISE_FP8 = "cozy.fp8-rowwise.native-leaf/1"
INT8_CONVROT = "cozy.int8-convrot256.native-leaf/1"


@dataclass(frozen=True, slots=True)
class PreQuantized:
    """A quantized activation as an encoded GEMM reads it (`accel/kernels.py:186-198`).

    `payload` holds the codes `[M, K]` (int8 or E4M3). `scale` holds the float32 scale of each
    row. `shape` is the 16-bit activation's shape, which fixes the output's leading dimensions.
    `provider` names the leaf family whose GEMM takes this geometry."""

    payload: Tensor
    scale: Tensor
    shape: tuple[int, ...]
    provider: str = ROWWISE_FP8


# ------------------------------------------------------------------------ S1: scopes


@dataclass(eq=False)
class _Scope:
    tensor: Tensor
    memo: dict[str, PreQuantized | None] = field(default_factory=dict)


_SCOPES: ContextVar[tuple[_Scope, ...]] = ContextVar("cozyq_operand_scopes", default=())


@contextmanager
def quantize_once(*tensors: Tensor | None) -> Iterator[None]:
    """Within the block, leaves reading one of `tensors` (by identity) quantize it once per
    provider between them (`accel/kernels.py:212-222`). None entries are ignored. The tensors
    must not be modified in place inside the block."""
    opened = tuple(_Scope(t) for t in tensors if t is not None)
    token = _SCOPES.set(_SCOPES.get() + opened)
    try:
        yield
    finally:
        _SCOPES.reset(token)


def _scoped(x: Tensor, provider: str, make: Make) -> tuple[bool, PreQuantized | None]:
    for scope in _SCOPES.get():
        if scope.tensor is x:
            if provider not in scope.memo:
                scope.memo[provider] = make()
            return True, scope.memo[provider]
    return False, None


# ------------------------------------------------------------ S4: learned reader groups

_GROUPS: weakref.WeakKeyDictionary[object, int] = weakref.WeakKeyDictionary()


def group_size(maker: object) -> int | None:
    """How many leaves were last seen reading one operand that `maker` made; None until a
    held operand of its making has been dropped."""
    return _GROUPS.get(maker)


def _learn(maker: object, readers: int) -> None:
    _GROUPS[maker] = max(_GROUPS.get(maker, 1), readers)


def _stamp(x: Tensor) -> tuple[object, ...]:
    """What must not change for a held operand to serve `x` again."""
    return (x._version, x.data_ptr(), tuple(x.shape), tuple(x.stride()), x.dtype)


# -------------------------------------------------------- S3/S5: the held operand


class _Hold:
    """One held operand: its input (weakly), the input's stamp, provider, operand, maker, the
    reads it served and the reads still expected (None while the maker's group is unknown)."""

    __slots__ = ("source", "stamp", "provider", "operand", "maker", "reads", "budget", "__weakref__")

    def __init__(self, owner: _Sharing, x: Tensor, provider: str, operand: PreQuantized,
                 maker: object, budget: int | None) -> None:  # fmt: skip
        me = weakref.ref(self)

        def died(_: object) -> None:
            hold = me()
            if hold is not None:
                owner.drop(hold)

        self.source = weakref.ref(x, died)
        self.stamp = _stamp(x)
        self.provider = provider
        self.operand: PreQuantized | None = operand
        self.maker = maker
        self.reads = 1
        self.budget = budget

    def matches(self, x: Tensor, provider: str) -> bool:
        return (self.operand is not None and provider == self.provider and self.source() is x
                and self.stamp == _stamp(x))  # fmt: skip


class _Sharing(threading.local):
    """The calling thread's sharing state: the held operand, and the group just read out (its
    input, stamp and maker), which grows by one if that input is asked for again next."""

    def __init__(self) -> None:
        self.hold: _Hold | None = None
        self.finished: tuple[Any, tuple[object, ...], object] | None = None

    def drop(self, hold: _Hold) -> None:
        if self.hold is hold:
            self.hold = None
        if hold.maker is not None:
            _learn(hold.maker, hold.reads)
        hold.operand = None
        hold.maker = None

    def ask(self, x: Tensor, provider: str, make: Make, consumer: object | None) -> PreQuantized | None:
        hold = self.hold
        if consumer is None or x.is_inference():  # S2
            if hold is not None:
                self.drop(hold)
            return None
        if hold is not None and hold.matches(x, provider):  # S3: a sibling reads it
            hold.reads += 1
            operand = hold.operand
            if hold.budget is not None:
                hold.budget -= 1
                if hold.budget <= 0:  # S4: the learned group has read it
                    self.finished = (hold.source, hold.stamp, hold.maker)
                    self.drop(hold)
            return operand
        if hold is not None:  # S5: another input or provider
            self.drop(hold)
        finished, self.finished = self.finished, None
        if finished is not None and finished[0]() is x and finished[1] == _stamp(x):
            _GROUPS[finished[2]] = _GROUPS.get(finished[2], 1) + 1  # one reader more than learned
        operand = make()
        if operand is None:
            return None
        group = _GROUPS.get(consumer)
        if group != 1:
            self.hold = _Hold(self, x, provider, operand, consumer, None if group is None else group - 1)
        return operand


_SHARING = _Sharing()


def shared_operand(
    x: Tensor, provider: str, make: Make, consumer: object | None = None
) -> PreQuantized | None:
    """`provider`'s operand for `x` (`accel/kernels.py:285-349`): made by `make()` for the first
    leaf that asks and read by the rest, by rules S1–S5 above. None when `make` declines or
    when nothing may be shared; the leaf then runs its op's one-call linear."""
    found, operand = _scoped(x, provider, make)
    if found:
        return operand
    return _SHARING.ask(x, provider, make, consumer)


# ----------------------------------------------------------------- producer hand-off


def _unbaked(module: object) -> object:
    """The base leaf of a composed layer whose update is baked into the base's bytes and that
    carries no hook of its own (`accel/kernels.py:385-395`): that leaf takes the operand."""
    while getattr(module, "_cozy_baked", False):
        hooked = getattr(module, "_forward_hooks", None) or getattr(module, "_forward_pre_hooks", None)
        base = getattr(module, "base_layer", None)
        if hooked or base is None:
            return module
        module = base
    return module


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
    """The rows a producer hands `consumers` — `activation(norm(x)·(1 + scale) + shift)` — rotated
    and quantized in one pass (`accel/kernels.py:352-382`), admitted by rules P1–P3: the first
    consumer's `int8_prologue` decides; None when it is not an int8.convrot-operand leaf."""
    leaves = tuple(_unbaked(c) for c in consumers)
    if not leaves or getattr(leaves[0], "operand", None) != INT8_CONVROT:
        return None
    return leaves[0].int8_prologue(x, leaves, norm, eps, scale, shift, activation, up)


def read(tensor: Any) -> Any:
    """A tensor launched by pointer, made readable first where it is a placeholder that binds
    on read (`accel/kernels.py:403-416`)."""
    bind = getattr(tensor, "_varena_read", None)
    return tensor if bind is None else bind()
