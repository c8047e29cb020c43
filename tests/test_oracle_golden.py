"""The oracle against the reference's own known-answer tests (CPU).

Every case in golden_cases.py cites the reference test it comes from. The
same cases run against the compiled reference (when it was built here) so
that the cases themselves are pinned, and against the HIP provider in
test_gpu_golden.py.
"""
import pytest

from golden_cases import CASES, CASE_IDS
from harness import ref_available, run_oracle, run_ref


@pytest.mark.parametrize("case", CASES, ids=CASE_IDS)
def test_oracle_matches_reference_kat(case):
    status, storages = run_oracle(case.kind, case.storages, case.views)
    case.check(status, storages)


@pytest.mark.skipif(not ref_available(),
                    reason="compiled reference (oracle/_ref) not built here")
@pytest.mark.parametrize("case", CASES, ids=CASE_IDS)
def test_compiled_reference_matches_kat_and_oracle(case):
    from conftest import m3
    if case.kind not in (m3.OP_ADD, m3.OP_MUL, m3.OP_CAST, m3.OP_COPY,
                         m3.OP_SOFTMAX, m3.OP_SNAKE1D, m3.OP_TANH,
                         m3.OP_GATED_SILU):
        pytest.skip("the reference has no such operation")
    status, storages = run_ref(case.kind, case.storages, case.views)
    case.check(status, storages)
    ostatus, ostorages = run_oracle(case.kind, case.storages, case.views)
    assert status == ostatus
    for a, b in zip(storages, ostorages):
        assert bytes(a) == bytes(b)
