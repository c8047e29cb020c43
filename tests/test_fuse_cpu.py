"""CPU checks of the session compiler's elementwise fusion planner
(m3.c_amd/csrc/host/m3_fuse.c) with tests/csrc/fuse_check.c built for the
host.

Each planned graph runs twice on the host: node by node with the
reference's per-element operation (load as F32, one F32 operation, round to
the output dtype; src/m3_op_execute_basic.c:61-77; CAST through F32 and
COPY as a raw copy, :11-59), and with every fused
group replaced by its program interpreted the way the kernel runs it. Every
value that has to reach memory must agree bit for bit, NaN payloads
included. Operands smaller than the output are broadcast along trailing
axes (read at e mod their count, the only kind that may fuse) or leading
ones. Values live in the slots of the session compiler's liveness plan, so
values whose lives do not overlap share bytes, and each program runs over
its elements in increasing and then decreasing order (a device's lanes run
in no fixed order). Nodes that never fuse (SOFTMAX, GATED_SILU) read values
between the groups. A plan with planted mistakes (a STORE of the wrong
register, SUB and DIV with swapped operands, periodic operands read without
their period) must be caught by the same comparison, and so must a planner
that is not told where values live (it would store over an operand other
elements still read) or what the non-fusing nodes read (it would keep
their inputs in registers only).
"""
import json
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [os.path.join(HERE, "csrc", "fuse_check.c"),
           os.path.join(ROOT, "m3.c_amd", "csrc", "host", "m3_fuse.c"),
           os.path.join(ROOT, "m3.c_amd", "csrc", "host", "m3_error.c")]
HEADERS = [os.path.join(ROOT, "m3.c_amd", "csrc", "host", "m3_fuse.h"),
           os.path.join(ROOT, "m3.c_amd", "csrc", "hip", "m3_numeric.h"),
           os.path.join(ROOT, "include", "m3_hip.h"),
           os.path.join(ROOT, "include", "m3_backend.h")]
TOOL = os.path.join(HERE, "_build", "fuse_check")


def build_checker():
    newest = max(os.path.getmtime(p) for p in SOURCES + HEADERS)
    if not os.path.exists(TOOL) or os.path.getmtime(TOOL) < newest:
        os.makedirs(os.path.dirname(TOOL), exist_ok=True)
        subprocess.run(
            ["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", "-Werror",
             "-ffp-contract=off", "-D_POSIX_C_SOURCE=200809L",
             "-I" + os.path.join(ROOT, "include"),
             "-I" + os.path.join(ROOT, "m3.c_amd", "csrc", "host"),
             "-I" + os.path.join(ROOT, "m3.c_amd", "csrc", "hip"),
             "-o", TOOL] + SOURCES, check=True)
    return TOOL


def run(*args, expect_ok=True):
    result = subprocess.run([build_checker(), *args], capture_output=True,
                            text=True, timeout=300)
    assert (result.returncode == 0) == expect_ok, result.stderr
    return json.loads(result.stdout)


def test_random_plans_match_node_by_node():
    for seed in (1, 2):
        r = run("random", "3000", str(seed))
        assert r["mismatches"] == 0
        assert r["stale_reads"] == 0
        assert r["structure_errors"] == 0
        assert r["unwritten_reads"] == 0
        # programs do read and write arrays that share a slot (same base,
        # same element size: each element is read before it is written)
        assert r["shared_slots"] > 500
        # the graphs do fuse, and fused temporaries stay out of memory
        assert r["groups"] > 5000
        assert r["internal_values"] > 5000
        assert r["compared_values"] > 50000
        # float CASTs, F32 COPYs and 16-bit values are fused too
        assert r["rounds"] > 1000
        assert r["rounding_ops"] > 1000
        assert r["narrow_operands"] > 1000
        # smaller operands broadcast along trailing axes are fused too
        assert r["periodic_operands"] > 1000


def test_planted_plan_mistakes_are_detected():
    r = run("random", "500", "3", "planted", expect_ok=False)
    assert r["mismatches"] > 100
    # a periodic operand without its period breaks the launcher's rules
    assert r["structure_errors"] > 100


def test_planner_that_ignores_shared_slots_is_detected():
    """Without address ranges the planner fuses runs whose stores land on
    a periodic or scalar operand, or on an operand of another element
    size, in a slot the liveness plan shares: one of the two element
    orders then reads overwritten bytes."""
    r = run("random", "3000", "1", "unaware", expect_ok=False)
    assert r["mismatches"] + r["stale_reads"] > 100


def test_planner_that_ignores_unfused_readers_is_detected():
    """A planner that does not see the inputs of SOFTMAX and GATED_SILU
    nodes keeps values they read in registers and never stores them."""
    r = run("random", "3000", "1", "blind", expect_ok=False)
    assert r["stale_reads"] > 100


def test_euler_graph_is_one_program():
    """30 CFG + Euler steps (6 nodes each, src/m3_flow_solver_math.c:
    36-135): one program, every temporary in registers, one store (the
    output), each of x and the 60 per-step tensors fetched about once."""
    r = run("euler", "30")
    assert r["mismatches"] == 0 and r["structure_errors"] == 0
    assert r["groups"] == 1
    assert r["first_group_nodes"] == 180
    assert r["stores"] == 1
    assert r["internal_values"] == 179
    # x, 30 vu, 30 vc, the three scalars and the output
    assert r["first_group_operands"] == 65
    assert 61 <= r["fetched_arrays"] <= 64


def test_long_chains_split_at_the_operand_limit():
    r = run("euler", "200")
    assert r["mismatches"] == 0 and r["structure_errors"] == 0
    assert r["groups"] == 2
    assert r["fused_nodes"] == 1200
