"""The HIP provider against the reference's known-answer tests (GPU).

Each case runs through m3_backend_execute on the HIP backend and must both
satisfy the reference's expected values and match the oracle byte for byte
(status and every storage, inputs included).
"""
import sys

import pytest

from golden_cases import CASES, CASE_IDS
from harness import HipFixture, run_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip(gpu):
    fixture = HipFixture()
    yield fixture
    fixture.close()


@pytest.mark.parametrize("case", CASES, ids=CASE_IDS)
def test_hip_matches_kat_and_oracle(hip, case):
    print("gpu case", case.name, flush=True, file=sys.stderr)
    status, storages, message = hip.run(case.kind, case.storages, case.views)
    case.check(status, storages)
    ostatus, ostorages = run_oracle(case.kind, case.storages, case.views)
    assert status == ostatus, message
    for a, b in zip(storages, ostorages):
        assert bytes(a) == bytes(b)
