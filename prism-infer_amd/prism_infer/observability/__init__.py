"""Profiling boundary of the ops, with the reference's API.

The API follows prism_infer/observability/performance.py:13-47:
``profile_region(name, *, cuda=True, metadata=None)`` returns a context
manager, a no-op until a provider pair is installed with
:func:`install_performance_provider` (non-callables raise TypeError), and
:func:`get_performance_profile_session` returns the installed session
provider's current session (None without one).  The ops keep the reference's
region names (``attention.kv_store.*``) so trace tooling keyed on them keeps
working.

Two ready-made region providers are included:

* :func:`record_function_region` -- a ``torch.profiler.record_function`` range,
  visible in ``torch.profiler`` traces;
* :func:`roctx_region` -- a ROCTX range (``torch.cuda.nvtx`` is ROCTX on
  ROCm), visible in ``rocprofv3 --marker-trace``; metadata is appended to the
  range name as ``key=value`` pairs.
"""

from __future__ import annotations

from contextlib import AbstractContextManager, contextmanager, nullcontext
from typing import Any, Callable, Iterator, Optional

ProfileRegionProvider = Callable[..., AbstractContextManager]
ProfileSessionProvider = Callable[[], Optional[Any]]

_region_provider: Optional[ProfileRegionProvider] = None
_session_provider: Optional[ProfileSessionProvider] = None


def install_performance_provider(*, profile_region_provider: ProfileRegionProvider,
                                 profile_session_provider: ProfileSessionProvider) -> None:
    """Install both providers; anything not callable (``None`` included) is a TypeError."""

    global _region_provider, _session_provider
    if not callable(profile_region_provider) or not callable(profile_session_provider):
        raise TypeError("install_performance_provider: both providers must be callables "
                        f"(got {type(profile_region_provider).__name__} and "
                        f"{type(profile_session_provider).__name__})")
    _region_provider = profile_region_provider
    _session_provider = profile_session_provider


def _reset_performance_providers() -> None:
    """Remove the installed providers (for tests); regions become no-ops again."""

    global _region_provider, _session_provider
    _region_provider = _session_provider = None


def profile_region(name: str, *, cuda: bool = True, metadata: Optional[dict] = None) -> AbstractContextManager:
    """A region of the installed provider, or a no-op context."""

    provider = _region_provider
    if provider is None:
        return nullcontext()
    return provider(name, cuda=cuda, metadata=metadata)


def get_performance_profile_session() -> Optional[Any]:
    provider = _session_provider
    return None if provider is None else provider()


def _label(name: str, metadata: Optional[dict]) -> str:
    if not metadata:
        return name
    return name + " " + " ".join(f"{k}={metadata[k]}" for k in sorted(metadata))


@contextmanager
def record_function_region(name: str, *, cuda: bool = True, metadata: Optional[dict] = None) -> Iterator[None]:
    """Region provider: a ``torch.profiler.record_function`` range."""

    import torch  # noqa: PLC0415

    with torch.profiler.record_function(_label(name, metadata)):
        yield


@contextmanager
def roctx_region(name: str, *, cuda: bool = True, metadata: Optional[dict] = None) -> Iterator[None]:
    """Region provider: a ROCTX range around the block (host-side markers;
    ``cuda`` is accepted for API compatibility, the range does not wait for
    the device)."""

    import torch  # noqa: PLC0415

    torch.cuda.nvtx.range_push(_label(name, metadata))
    try:
        yield
    finally:
        torch.cuda.nvtx.range_pop()


__all__ = [
    "get_performance_profile_session",
    "install_performance_provider",
    "profile_region",
    "record_function_region",
    "roctx_region",
]
