"""The profiling boundary: the reference's provider API and the shipped providers.

API semantics follow prism_infer/observability/performance.py:13-47 (no-op
without providers, TypeError for non-callables, the session provider's value
returned as is).  The store op's region names follow
prism_infer/ops/kv_cache_store.py:340-347 with this build's backend name.
"""

from __future__ import annotations

from contextlib import contextmanager, nullcontext

import pytest
import torch

from prism_infer import observability as obs
from prism_infer.ops.kv_cache_store import _store_profile_region


@pytest.fixture(autouse=True)
def _no_provider():
    obs._reset_performance_providers()
    yield
    obs._reset_performance_providers()


def test_default_is_a_noop():
    assert isinstance(obs.profile_region("x"), nullcontext)
    assert obs.get_performance_profile_session() is None


def test_non_callable_providers_raise():
    with pytest.raises(TypeError):
        obs.install_performance_provider(profile_region_provider="nope", profile_session_provider=lambda: None)
    with pytest.raises(TypeError):
        obs.install_performance_provider(profile_region_provider=lambda *a, **k: nullcontext(),
                                         profile_session_provider=3)
    with pytest.raises(TypeError):
        obs.install_performance_provider(profile_region_provider=None, profile_session_provider=None)


def test_installed_providers_receive_name_cuda_and_metadata():
    seen = []

    @contextmanager
    def region(name, *, cuda=True, metadata=None):
        seen.append(("enter", name, cuda, metadata))
        yield
        seen.append(("exit", name))

    session = object()
    obs.install_performance_provider(profile_region_provider=region, profile_session_provider=lambda: session)
    with obs.profile_region("attention.kv_store.hip_scaled_fp8", cuda=False, metadata={"tokens": 4}):
        seen.append(("body",))
    assert seen == [("enter", "attention.kv_store.hip_scaled_fp8", False, {"tokens": 4}), ("body",),
                    ("exit", "attention.kv_store.hip_scaled_fp8")]
    assert obs.get_performance_profile_session() is session


def test_record_function_provider_shows_in_torch_profiler():
    obs.install_performance_provider(profile_region_provider=obs.record_function_region,
                                     profile_session_provider=lambda: None)
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
        with obs.profile_region("attention.kv_store.hip", metadata={"tokens": 7}):
            torch.ones(4).sum()
    names = {e.name for e in prof.events()}
    assert "attention.kv_store.hip tokens=7" in names


def test_store_region_names():
    fp8 = torch.empty(1, dtype=torch.float8_e4m3fn)
    bf16 = torch.empty(1, dtype=torch.bfloat16)
    assert _store_profile_region(True, fp8) == "attention.kv_store.hip_scaled_fp8"
    assert _store_profile_region(False, fp8) == "attention.kv_store.hip_fp8"
    assert _store_profile_region(False, bf16) == "attention.kv_store.hip"
