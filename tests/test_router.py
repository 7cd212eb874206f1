"""Router: the reference's known-answer tests (tests/test_kernel_router.py:7-20) against the build
and the oracle, plus the frozen-dataclass surface (router.py:8-17)."""
import dataclasses
import json
import os

import pytest

from dynakv_amd.kernels.router import KernelPolicy
from oracle import router as oracle_router

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "router_kat.json")


def test_default_kernel_boundary():
    policy = KernelPolicy()
    assert policy.select(0) == "short_fused"
    assert policy.select(499) == "short_fused"
    assert policy.select(500) == "long_two_stage"


def test_custom_kernel_boundary():
    policy = KernelPolicy(switch_tokens=128)
    assert policy.select(127) == "short_fused"
    assert policy.select(128) == "long_two_stage"


def test_negative_cache_length_is_rejected():
    with pytest.raises(ValueError):
        KernelPolicy().select(-1)
    with pytest.raises(ValueError):
        oracle_router.select(-1)


def test_golden_vectors_build_and_oracle():
    with open(GOLDEN) as f:
        cases = json.load(f)["cases"]
    assert len(cases) >= 5
    for c in cases:
        pol = KernelPolicy(**({"switch_tokens": c["switch_tokens"]} if "switch_tokens" in c else {}))
        assert pol.select(c["cache_length"]) == c["expect"], c
        assert oracle_router.select(c["cache_length"], pol.switch_tokens) == c["expect"], c


def test_policy_is_frozen_dataclass():
    pol = KernelPolicy()
    assert dataclasses.is_dataclass(pol)
    assert pol.switch_tokens == 500
    with pytest.raises(dataclasses.FrozenInstanceError):
        pol.switch_tokens = 10  # type: ignore[misc]


def test_router_sweep_matches_oracle():
    for sw in (1, 64, 128, 500, 4096):
        pol = KernelPolicy(switch_tokens=sw)
        for L in list(range(0, 600)) + [sw - 1, sw, sw + 1, 16384]:
            if L < 0:
                continue
            assert pol.select(L) == oracle_router.select(L, sw)
