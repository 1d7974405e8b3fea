"""WMN1 model sessions (Stack and Grid roots) on the GPU against the oracle.

Stack forward chains the flattened children (stack.cpp:470-494); a Grid runs
its cells serially in (z, y, x, l) hop order, skipping disabled cells and
reading remote-link inputs from recorded posts (runtime/forward.cpp:98-156).
"""
import numpy as np
import pytest

import pywelvet as pw
from test_gpu_dense import rel_l2, tol

pytestmark = pytest.mark.gpu


def build_stack(layers, root=0, dims=(1, 1, 1, 1), cells=None):
    """layers: list (per child) of lists of (dtype, W, act). Stack root: one
    NestedStack child per entry; Grid root: one child per cell."""
    w = pw.Wire()
    w.u32(0x314E4D57)
    w.i32(root, len(layers), *dims)
    for child in layers:
        w.i32(19, len(child))
        for dt, W, act in child:
            pw.dense_child(w, W.shape[1], W.shape[0], act, dt, W)
    pw.empty_controls(w)
    for child in layers:
        pw.empty_controls(w)
        for _ in child:
            pw.empty_controls(w)
    stores = [(dt, W) for child in layers for dt, W, _ in child]
    w.i32(len(stores))
    orc = __import__("oracle_lib").Oracle()
    for dt, W in stores:
        pw.store_payload(w, dt, W.shape[0], W.shape[1], orc.pack(dt, W))
    if root == 2:
        for c in cells:
            w.i32(*c)
    return w.bytes()


def oracle_chain(oracle, seq, x, scheme=0):
    cur = x
    for dt, W, act in seq:
        rows, cols = W.shape
        native, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
        Wd = oracle.dequant(dt, scheme, rows, cols, native, rs, blk)
        _, cur = oracle.dense(Wd, cur, act)
    return cur


def test_stack_of_three_dense(gpu, oracle):
    rng = np.random.default_rng(5)
    dims = [96, 128, 64, 80]
    layers = [(dt, (rng.standard_normal((dims[i + 1], dims[i])) * 2).astype(np.float32), act)
              for i, (dt, act) in enumerate([(4, 0), (16, -1), (4, 1)])]
    x = rng.standard_normal((3, 96)).astype(np.float32)
    m = pw.ModelSession(build_stack([layers]))
    y = m.forward(x)
    assert y.shape == (3, 80)
    assert rel_l2(y, oracle_chain(oracle, layers, x)) <= tol(3, chain=3)
    snap = m.export()
    assert snap[:4] == b"NWS1" and int(np.frombuffer(snap[4:8], "<i4")[0]) == 3
    m.close()


def test_stack_requantized_with_scheme(gpu, oracle):
    rng = np.random.default_rng(6)
    layers = [(dt, (rng.standard_normal((64, 64)) / 8).astype(np.float32), -1)
              for dt in (4, 16, 4)]
    x = rng.standard_normal((2, 64)).astype(np.float32)
    for scheme in (1, 2, 3):
        m = pw.ModelSession(build_stack([layers]), scheme=scheme)
        assert rel_l2(m.forward(x), oracle_chain(oracle, layers, x, scheme)) <= tol(2, chain=3)
        m.close()


def test_grid_hop_order_disabled_and_remote(gpu, oracle):
    rng = np.random.default_rng(7)
    W = [(rng.standard_normal((32, 32)) / 4).astype(np.float32) for _ in range(4)]
    cells_layers = [[(4, W[i], -1)] for i in range(4)]
    # 2x2x1x1 grid: cell 2 disabled; cell 3 reads cell 0's post (remote link)
    cells = [(1, 0, 0, 0, 0, 0), (1, 0, 0, 0, 0, 0), (0, 0, 0, 0, 0, 0), (1, 1, 0, 0, 0, 0)]
    m = pw.ModelSession(build_stack(cells_layers, root=2, dims=(2, 2, 1, 1), cells=cells))
    x = rng.standard_normal((2, 32)).astype(np.float32)
    y = m.forward(x)
    p0 = oracle_chain(oracle, cells_layers[0], x)
    want = oracle_chain(oracle, cells_layers[3], p0)
    assert rel_l2(y, want) <= tol(2, chain=2)
    m.close()


def test_c1_volume_single_dense_cell(gpu, oracle):
    """1x1x1 volume, one Dense 512->512 E4M3 with a per-tensor scale, batch 1."""
    W = pw.normal(pw.seed_for(1), 512 * 512, 1 / np.sqrt(512)).reshape(512, 512)
    x = pw.normal(pw.seed_for(1) + 500, 512).reshape(1, 512)
    layers = [[(4, W, -1)]]
    m = pw.ModelSession(build_stack(layers, root=2, dims=(1, 1, 1, 1), cells=[(1, 0, 0, 0, 0, 0)]),
                        scheme=1)
    y = m.forward(x)
    assert rel_l2(y, oracle_chain(oracle, layers[0], x, scheme=1)) <= 1e-5
    m.close()


def test_repeated_forwards_reuse_device_buffers(gpu, oracle):
    """A model keeps its pass buffers and workspace between forwards: batches
    that take every path (GEMV 1, small-batch matrix cores 3, K-split 16,
    large tiles 40), in an order that grows and shrinks them, all match."""
    rng = np.random.default_rng(9)
    layers = [(dt, (rng.standard_normal((256, 256)) / 16).astype(np.float32), act)
              for dt, act in ((4, -1), (16, 1), (5, -1))]
    m = pw.ModelSession(build_stack([layers]), scheme=2)
    for batch in (1, 3, 16, 40, 3, 40, 1):
        x = rng.standard_normal((batch, 256)).astype(np.float32)
        y = m.forward(x)
        assert y.shape == (batch, 256)
        assert rel_l2(y, oracle_chain(oracle, layers, x, scheme=2)) <= tol(batch, chain=3), batch
    m.close()


@pytest.mark.parametrize("scheme", [2, 3])
def test_grid_chain_matches_layer_by_layer(gpu, oracle, scheme):
    """A grid of two Stack cells run as one chain gives the bits of running
    each layer as its own session (same kernels: split-K products at 200
    rows, 56 padding rows). Layers: 1024 -> 1024 (SiLU) -> 1024 -> 512 |
    512 -> 768 -> 256."""
    rng = np.random.default_rng(10 + scheme)
    widths = [1024, 1024, 1024, 512, 768, 256]
    kinds = [(4, 1), (16, -1), (5, -1), (4, 0), (16, -1)]
    seq = [(dt, (rng.standard_normal((widths[i + 1], widths[i])) / np.sqrt(widths[i])).astype(np.float32), act)
           for i, (dt, act) in enumerate(kinds)]
    cells = [(1, 0, 0, 0, 0, 0), (1, 0, 0, 0, 0, 0)]
    m = pw.ModelSession(build_stack([seq[:3], seq[3:]], root=2, dims=(2, 1, 1, 1), cells=cells),
                        scheme=scheme)
    x = rng.standard_normal((200, 1024)).astype(np.float32)
    y = m.forward(x)
    cur = x
    for dt, W, act in seq:
        s = pw.DenseSession(200, W.shape[1], W.shape[0], act, dt, scheme, W)
        _, cur = s.execute(cur)
        s.close()
    assert np.array_equal(y, cur)
    assert rel_l2(y, oracle_chain(oracle, seq, x, scheme)) <= tol(200, chain=5)
    y2 = m.forward(x)  # a second pass over the same buffers
    assert np.array_equal(y2, y)
    m.close()
