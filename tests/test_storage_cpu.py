"""The storage contract on the host backend (CPU): see
tests/storage_contract.py."""
from storage_contract import check_storage_contract


def test_host_backend_storage_contract():
    check_storage_contract("m3_backend_create_host", device_memory=False)
