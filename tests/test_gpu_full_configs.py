"""The five workloads at their full sizes through the public API (GPU).

Each runs as a session on the HIP provider and is compared bit for bit over
the whole output: with the oracle (the reference's algorithms restated in C,
run in pieces on parallel threads) for softmax, the casts and Snake1d, and
with the same float32 operations in numpy for MUL and the Euler graph, whose
elementwise IEEE operations numpy performs identically.

  C1  MUL x[8,1024,1536] * c[1536]
  C2  causal softmax [16,1024,1024], logits ~ N(0, 3)
  C3  F32 <-> F16/BF16 casts of [4096,4096] with 5% special values
  C4  Snake1d x[2,1536,65536], alpha[1,1536,1]
  C5  the 30-step Euler CFG graph on [2,4096,1536]
"""
import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from conftest import m3
from harness import ViewSpec, as_bytes, run_oracle

pytestmark = pytest.mark.gpu

THREADS = 16


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype.itemsize == 4
                                        else np.uint16)


def run_graph(graph, feeds, outputs):
    session = m3.Session(graph)
    graph.free()
    try:
        for node in range(session.plan().node_count):
            assert session.provider(node) == m3.PROVIDER_HIP
        for value, array in feeds:
            session.write(value, array)
        session.run()
        return [session.read(value, np.zeros(shape, dtype))
                for value, shape, dtype in outputs]
    finally:
        session.free()


def oracle_pieces(kind, pieces):
    """Runs the oracle over independent pieces in parallel (ctypes releases
    the GIL); each piece is (storages, views, index of the output)."""
    def one(piece):
        storages, views, out = piece
        status, result = run_oracle(kind, storages, views)
        assert status == m3.OK
        return result[out]

    with ThreadPoolExecutor(THREADS) as pool:
        return list(pool.map(one, pieces))


def test_c1_mul_full(gpu):
    print("gpu case C1 full", file=sys.stderr, flush=True)
    shape = (8, 1024, 1536)
    x = m3.rng_fill("uniform", int(np.prod(shape)), seed=0, a=-1.0,
                    b=1.0).reshape(shape)
    c = m3.rng_fill("normal", shape[-1], seed=0, sequence=1, a=1.0)
    g = m3.Graph()
    vx = g.add_value(m3.INPUT, m3.F32, shape)
    vc = g.add_value(m3.CONSTANT, m3.F32, shape[-1:])
    vy = g.add_value(m3.OUTPUT, m3.F32, shape)
    g.set_constant(vc, c)
    g.add_node(m3.OP_MUL, [vx, vc], [vy])
    (y,) = run_graph(g, [(vx, x)], [(vy, shape, np.float32)])
    assert np.array_equal(bits(y), bits((x * c).astype(np.float32)))


def test_c2_softmax_full(gpu):
    print("gpu case C2 full", file=sys.stderr, flush=True)
    heads, n = 16, 1024
    s = m3.rng_fill("normal", heads * n * n, seed=0, a=3.0).reshape(heads, n,
                                                                    n)
    s[:, np.triu(np.ones((n, n), bool), k=1)] = -np.inf
    g = m3.Graph()
    vi = g.add_value(m3.INPUT, m3.F32, s.shape)
    vo = g.add_value(m3.OUTPUT, m3.F32, s.shape)
    g.add_node(m3.OP_SOFTMAX, [vi], [vo])
    (p,) = run_graph(g, [(vi, s)], [(vo, s.shape, np.float32)])
    pieces = [([as_bytes(s[h]), np.zeros(n * n * 4, np.uint8)],
               [ViewSpec(0, m3.F32, (n, n)), ViewSpec(1, m3.F32, (n, n))], 1)
              for h in range(heads)]
    expected = oracle_pieces(m3.OP_SOFTMAX, pieces)
    for h in range(heads):
        assert np.array_equal(bits(p[h]), expected[h].view(np.uint32)
                              .reshape(n, n)), "head %d" % h


def cast_source(src_dtype, n=4096, seed=7):
    rng = np.random.default_rng(seed)
    values = (rng.standard_normal(n * n) * 1000).astype(np.float32)
    raw = values.view(np.uint32).copy()
    pick = rng.random(n * n) < 0.05
    specials = np.array([0x00000001, 0x007fffff, 0x80000000, 0x00000000,
                         0x7f800000, 0xff800000, 0x7fc00001, 0x7f800123,
                         0xffa00000], np.uint32)
    raw[pick] = specials[rng.integers(len(specials), size=int(pick.sum()))]
    f32 = raw.view(np.float32).reshape(n, n)
    if src_dtype == m3.F16:
        return f32.astype(np.float16).view(np.uint16)
    if src_dtype == m3.BF16:
        return (f32.view(np.uint32) >> 16).astype(np.uint16)
    return f32


@pytest.mark.parametrize("pair", [(m3.F32, m3.F16), (m3.F16, m3.F32),
                                  (m3.F32, m3.BF16), (m3.BF16, m3.F32)],
                         ids=["f32_f16", "f16_f32", "f32_bf16", "bf16_f32"])
def test_c3_cast_full(gpu, pair):
    print("gpu case C3 full", pair, file=sys.stderr, flush=True)
    src_dtype, dst_dtype = pair
    src = cast_source(src_dtype)
    n = src.shape[0]
    out_np = np.float32 if dst_dtype == m3.F32 else np.uint16
    g = m3.Graph()
    vi = g.add_value(m3.INPUT, src_dtype, src.shape)
    vo = g.add_value(m3.OUTPUT, dst_dtype, src.shape)
    g.add_node(m3.OP_CAST, [vi], [vo])
    (got,) = run_graph(g, [(vi, src)], [(vo, src.shape, out_np)])
    rows = n // THREADS
    size = np.dtype(out_np).itemsize
    pieces = [([as_bytes(src[r:r + rows]), np.zeros(rows * n * size,
                                                    np.uint8)],
               [ViewSpec(0, src_dtype, (rows, n)),
                ViewSpec(1, dst_dtype, (rows, n))], 1)
              for r in range(0, n, rows)]
    expected = np.concatenate([e.view(out_np) for e in
                               oracle_pieces(m3.OP_CAST, pieces)])
    assert np.array_equal(bits(got).reshape(-1), bits(expected))


def test_c4_snake_full(gpu):
    print("gpu case C4 full", file=sys.stderr, flush=True)
    shape = (2, 1536, 65536)
    x = m3.rng_fill("normal", int(np.prod(shape)), seed=0,
                    a=1.0).reshape(shape)
    alpha = m3.rng_fill("uniform", shape[1], seed=0, sequence=1, a=0.1,
                        b=2.0).reshape(1, shape[1], 1)
    g = m3.Graph()
    vx = g.add_value(m3.INPUT, m3.F32, shape)
    va = g.add_value(m3.CONSTANT, m3.F32, alpha.shape)
    vy = g.add_value(m3.OUTPUT, m3.F32, shape)
    g.set_constant(va, alpha)
    g.add_node(m3.OP_SNAKE1D, [vx, va], [vy])
    (y,) = run_graph(g, [(vx, x)], [(vy, shape, np.float32)])
    block = 96
    pieces = []
    for b in range(shape[0]):
        for c in range(0, shape[1], block):
            piece = np.ascontiguousarray(x[b:b + 1, c:c + block])
            a = np.ascontiguousarray(alpha[:, c:c + block])
            pieces.append(([as_bytes(piece), as_bytes(a),
                            np.zeros(piece.nbytes, np.uint8)],
                           [ViewSpec(0, m3.F32, piece.shape),
                            ViewSpec(1, m3.F32, a.shape),
                            ViewSpec(2, m3.F32, piece.shape)], 2))
    expected = oracle_pieces(m3.OP_SNAKE1D, pieces)
    k = 0
    for b in range(shape[0]):
        for c in range(0, shape[1], block):
            assert np.array_equal(
                bits(y[b:b + 1, c:c + block]).reshape(-1),
                expected[k].view(np.uint32)), "batch %d channel %d" % (b, c)
            k += 1


def test_c5_euler_full(gpu):
    print("gpu case C5 full", file=sys.stderr, flush=True)
    shape = (2, 4096, 1536)
    count = int(np.prod(shape))
    steps = 30
    rng = m3.rng_new(0, 0)
    x0 = m3.rng_fill("normal", count, seed=0, a=1.0, rng=rng).reshape(shape)
    scale = np.float32(3.0)
    dt = np.float32(1.0 / 30.0)
    g = m3.Graph()
    vx = g.add_value(m3.INPUT, m3.F32, shape)
    consts = {}
    for name, value in (("minus_one", -1.0), ("scale", scale), ("dt", dt)):
        vid = g.add_value(m3.CONSTANT, m3.F32, (1,))
        g.set_constant(vid, np.array([value], np.float32))
        consts[name] = vid
    current = vx
    expected = x0.copy()
    for k in range(steps):
        vu_data = m3.rng_fill("normal", count, seed=0, a=1.0,
                              rng=rng).reshape(shape)
        vc_data = m3.rng_fill("normal", count, seed=0, a=1.0,
                              rng=rng).reshape(shape)
        vu = g.add_value(m3.CONSTANT, m3.F32, shape)
        vc = g.add_value(m3.CONSTANT, m3.F32, shape)
        g.set_constant(vu, vu_data)
        g.set_constant(vc, vc_data)
        t = [g.add_value(m3.TEMPORARY, m3.F32, shape) for _ in range(5)]
        nxt = g.add_value(m3.OUTPUT if k == steps - 1 else m3.TEMPORARY,
                          m3.F32, shape)
        g.add_node(m3.OP_MUL, [vu, consts["minus_one"]], [t[0]])
        g.add_node(m3.OP_ADD, [vc, t[0]], [t[1]])
        g.add_node(m3.OP_MUL, [t[1], consts["scale"]], [t[2]])
        g.add_node(m3.OP_ADD, [vu, t[2]], [t[3]])
        g.add_node(m3.OP_MUL, [t[3], consts["dt"]], [t[4]])
        g.add_node(m3.OP_ADD, [current, t[4]], [nxt])
        current = nxt
        a = vu_data * np.float32(-1.0)
        a = vc_data + a
        a = a * scale
        v = vu_data + a
        expected = expected + v * dt
        assert expected.dtype == np.float32
    (y,) = run_graph(g, [(vx, x0)], [(current, shape, np.float32)])
    assert np.array_equal(bits(y), bits(expected))
