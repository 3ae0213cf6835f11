"""Drop-in for the reference module ``lazy_recall._host`` (csrc/host.cpp:5-18).

``register_host(address, bytes)`` page-locks caller-owned host memory (the recall
transport's POSIX shared-memory rings, src/lazy_recall/recall/transport.py:16-44) so that
copies between it and the GPU run asynchronously; ``unregister_host(address)`` releases it.
Failures raise RuntimeError, as the reference's TORCH_CHECK does.
"""

from __future__ import annotations

from . import _lib


def register_host(address: int, bytes: int) -> None:  # noqa: A002 (reference argument name)
    _lib.call("lr_register_host", int(address), int(bytes))


def unregister_host(address: int) -> None:
    _lib.call("lr_unregister_host", int(address))
