"""No-op profiling facade with the reference's region API.

Mirrors ``profile_region(name, cuda=True, metadata=None)`` of
prism_infer/observability/performance.py:31-42: a context manager that does
nothing unless a provider is installed with :func:`install_profile_provider`.
The ops keep the reference's region names (``attention.kv_store.*``,
``attention.decode.*``) so existing trace tooling keeps working.
"""

from __future__ import annotations

from contextlib import nullcontext
from typing import Any, Callable

_PROVIDER: Callable[..., Any] | None = None


def install_profile_provider(provider: Callable[..., Any] | None) -> None:
    """Install (or clear with ``None``) a callable returning a context manager."""

    global _PROVIDER
    _PROVIDER = provider


def profile_region(name: str, cuda: bool = True, metadata: dict | None = None):
    if _PROVIDER is None:
        return nullcontext()
    return _PROVIDER(name, cuda=cuda, metadata=metadata)


__all__ = ["install_profile_provider", "profile_region"]
