"""Error types mirroring esp's `InferError` (crates/esp/src/infer/provider.rs:160-183).

Each variant is a Python exception subclass; the C ABI reports the same
variants as `esp_status` codes (include/esp_hip.h), and `raise_for_status`
maps a code plus the thread-local message back to the matching exception.
"""
from __future__ import annotations


class InferError(Exception):
    """Base of every error the decoder raises (provider.rs:160)."""

    code = 0


class PromptTooLong(InferError):
    """provider.rs:162 `PromptTooLong { length, limit }`."""

    code = 1

    def __init__(self, length: int, limit: int):
        super().__init__(f"prompt too long: {length} > {limit}")
        self.length = length
        self.limit = limit


class ModelNotLoaded(InferError):
    """provider.rs:164"""

    code = 2


class Interrupted(InferError):
    """provider.rs:166"""

    code = 3


class Backend(InferError):
    """provider.rs:168 — the runtime (here: HIP) failed."""

    code = 4


class StageUnavailable(InferError):
    """provider.rs:171"""

    code = 5


class InvalidRequest(InferError):
    """provider.rs:173 — empty input, over-window input, bad ids, ..."""

    code = 6


class InvalidConfig(InferError):
    """provider.rs:175"""

    code = 7


class InvalidWeights(InferError):
    """provider.rs:177"""

    code = 8


class Unsupported(InferError):
    """provider.rs:182 `Unsupported { feature, detail }`."""

    code = 9

    def __init__(self, feature: str, detail: str):
        super().__init__(f"unsupported {feature}: {detail}")
        self.feature = feature
        self.detail = detail


_BY_CODE = {
    cls.code: cls
    for cls in (ModelNotLoaded, Interrupted, Backend, StageUnavailable, InvalidRequest,
                InvalidConfig, InvalidWeights)
}


def raise_for_status(code: int, message: str) -> None:
    """Raise the exception matching an `esp_status` code (0 = success)."""
    if code == 0:
        return
    if code == PromptTooLong.code:
        parts = message.rsplit(" ", 3)
        try:
            raise PromptTooLong(int(parts[-3]), int(parts[-1]))
        except (ValueError, IndexError):
            raise InvalidRequest(message) from None
    if code == Unsupported.code:
        feature, _, detail = message.partition(": ")
        raise Unsupported(feature, detail)
    raise _BY_CODE.get(code, Backend)(message)
