"""The storage contract on the HIP backend (GPU): device memory reached
only through stream-ordered copies, after the reference's test of its GPU
backend (tests/test_metal_runtime.c:40-172). See
tests/storage_contract.py."""
import pytest

from storage_contract import check_storage_contract

pytestmark = pytest.mark.gpu


def test_hip_backend_storage_contract(gpu):
    check_storage_contract("m3_backend_create_hip", device_memory=True)
