"""WMN1 model sessions (Stack and Grid roots) on the GPU against the oracle.

Stack forward chains the flattened children (stack.cpp:470-494); a Grid runs
its cells serially in (z, y, x, l) hop order, skipping disabled cells and
reading remote-link inputs from recorded posts (runtime/forward.cpp:98-156).
"""
import numpy as np
import pytest

import pywelvet as pw
from test_gpu_dense import TOL_CONTRACT, rel_l2, tol

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


@pytest.mark.parametrize("scheme", [2, 3, 2 | 16, 3 | 32])
def test_grid_chain_matches_layer_by_layer(gpu, oracle, scheme):
    """A grid of two Stack cells run as one chain gives the bits of running
    each layer as its own session (split-K products at 200 rows, 56 padding
    rows). Within a cell the chain fuses the next layer's activation split
    into each K-split reduce (no split launch between the products), which
    must not change a bit. Layers: 1024 -> 1024 (SiLU) -> 1024 -> 512 |
    512 -> 768 -> 256; three activation terms (FP6), two (bit 16) and one
    (bit 32)."""
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
    err = rel_l2(y, oracle_chain(oracle, seq, x, scheme & 15))
    if scheme & 32:  # one E4M3 term: ~2.7e-2 per product, outside the contract bound
        assert err <= 0.15
    elif scheme & 16:  # two E4M3 terms: ~6.3e-4 per product
        assert err <= 5 * TOL_CONTRACT
    else:
        assert err <= tol(200, chain=5)
    y2 = m.forward(x)  # a second pass over the same buffers
    assert np.array_equal(y2, y)
    m.close()


def parse_nws1(snap):
    """Stores of an NWS1 snapshot: (dtype, rows, cols, scale, native bytes)."""
    stores, _ = pw.parse_snapshot(snap)
    return [(dt, rows, cols, scale, native) for dt, _, rows, cols, scale, _, native, _ in stores]


def _segment_layers(rng):
    dims = [96, 128, 64, 80]
    return [(dt, (rng.standard_normal((dims[i + 1], dims[i])) / np.sqrt(dims[i])).astype(np.float32), act)
            for i, (dt, act) in enumerate([(4, 0), (16, -1), (5, 1)])]


@pytest.mark.parametrize("scheme,batch", [(0, 3), (2, 40), (3, 1)])
def test_segment_backward_matches_layer_by_layer(gpu, oracle, scheme, batch):
    """welvet_model_backward of a Stack (model_session.cpp:435-455): the
    input gradient and the concatenated dW are the bits of running the Dense
    NormalBP leaf layer by layer in reverse on the forward's activations
    (same kernels), and match the oracle's chain within the chained bound."""
    rng = np.random.default_rng(20 + scheme + batch)
    layers = _segment_layers(rng)
    m = pw.ModelSession(build_stack([layers]), scheme=scheme)
    x = rng.standard_normal((batch, 96)).astype(np.float32)
    gy = rng.standard_normal((batch, 80)).astype(np.float32)
    gx, dw = m.backward(x, gy)
    assert gx.shape == (batch, 96) and dw.shape == (1, 128 * 96 + 64 * 128 + 80 * 64)
    ins, cur = [], x
    for dt, W, act in layers:
        ins.append(cur)
        _, cur = pw.dense_forward(batch, W.shape[1], W.shape[0], act, dt, scheme, W, cur)
    g, parts = gy, []
    for (dt, W, act), xi in reversed(list(zip(layers, ins))):
        _, _, g, dwi, _, _ = pw.dense_normalbp(batch, W.shape[1], W.shape[0], act, dt, scheme, W, xi, g)
        parts.insert(0, dwi.ravel())
    assert np.array_equal(gx, g)
    assert np.array_equal(dw.ravel(), np.concatenate(parts))
    # the oracle's chain: its own forward, then the backward in reverse
    Wd = []
    for dt, W, _ in layers:
        native, rs, blk = oracle.quantize(dt, scheme, W.shape[0], W.shape[1], W)
        Wd.append(oracle.dequant(dt, scheme, W.shape[0], W.shape[1], native, rs, blk))
    ins_o, pres_o, cur = [], [], x
    for (dt, W, act), Wq in zip(layers, Wd):
        ins_o.append(cur)
        pre, cur = oracle.dense(Wq, cur, act)
        pres_o.append(pre)
    g, parts = gy, []
    for (dt, W, act), Wq, xi, pre in reversed(list(zip(layers, Wd, ins_o, pres_o))):
        _, g, dwi = oracle.backward(Wq, g, pre, xi, act)
        parts.insert(0, dwi.ravel())
    assert rel_l2(gx, g) <= 1e-4 and rel_l2(dw.ravel(), np.concatenate(parts)) <= 1e-4
    m.close()


@pytest.mark.parametrize("scheme", [0, 2, 3])
def test_segment_sgd_requantizes_every_store(gpu, oracle, scheme):
    """welvet_model_apply_sgd (model_session.cpp:494-507, stack.cpp:561-580):
    each Dense store becomes quantize(f32(f64(dequant(W)) - lr * f64(dW slice)))
    with the model's scheme; the exported payloads match the oracle's bytes."""
    rng = np.random.default_rng(30 + scheme)
    layers = _segment_layers(rng)
    m = pw.ModelSession(build_stack([layers]), scheme=scheme)
    x = rng.standard_normal((8, 96)).astype(np.float32)
    _, dw = m.backward(x, rng.standard_normal((8, 80)).astype(np.float32))
    lr = 0.25
    m.apply_sgd(dw, lr)
    snap = m.export()
    assert all(sc == scheme for _, sc, *_ in pw.parse_snapshot(snap)[0])
    stores = parse_nws1(snap)
    off = 0
    for (dt, W, _), (sdt, rows, cols, _, native) in zip(layers, stores):
        n = W.size
        nat, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
        Wq = oracle.dequant(dt, scheme, rows, cols, nat, rs, blk)
        nxt = oracle.sgd(Wq, dw.ravel()[off:off + n].reshape(W.shape), lr)
        nat2, _, _ = oracle.quantize(dt, scheme, rows, cols, nxt)
        assert sdt == dt and np.array_equal(native, nat2), dt
        off += n
    m.close()


def test_segment_training_errors(gpu):
    rng = np.random.default_rng(40)
    layers = _segment_layers(rng)
    m = pw.ModelSession(build_stack([layers]))
    x = rng.standard_normal((2, 96)).astype(np.float32)
    with pytest.raises(pw.WelvetError) as e:  # gradient of the wrong shape
        m.backward(x, np.zeros((2, 79), np.float32))
    assert e.value.code == 1
    with pytest.raises(pw.WelvetError) as e:  # dW of the wrong size
        m.apply_sgd(np.zeros((1, 7), np.float32), 0.1)
    assert e.value.code == 1
    with pytest.raises(pw.WelvetError) as e:
        m.apply_sgd(np.zeros((1, 7), np.float32), float("nan"))
    assert e.value.code == 1
    m.close()
    W = (rng.standard_normal((32, 32)) / 4).astype(np.float32)
    g = pw.ModelSession(build_stack([[(4, W, -1)]], root=2, dims=(1, 1, 1, 1),
                                    cells=[(1, 0, 0, 0, 0, 0)]))
    with pytest.raises(pw.WelvetError) as e:  # segment calls take Stack roots
        g.backward(np.zeros((1, 32), np.float32), np.zeros((1, 32), np.float32))
    assert e.value.code == 1
    g.close()


@pytest.mark.parametrize("batch", [3, 40])
def test_segment_forward_pair(gpu, batch):
    """welvet_model_forward_pair: the last op's pre-activation and the output,
    the bits of the layers run one by one."""
    rng = np.random.default_rng(50 + batch)
    layers = _segment_layers(rng)  # last op SiLU: pre and post differ
    m = pw.ModelSession(build_stack([layers]), scheme=2)
    x = rng.standard_normal((batch, 96)).astype(np.float32)
    pre, post = m.forward_pair(x)
    cur = x
    for dt, W, act in layers:
        want_pre, cur = pw.dense_forward(batch, W.shape[1], W.shape[0], act, dt, 2, W, cur)
    assert np.array_equal(pre, want_pre) and np.array_equal(post, cur)
    assert not np.array_equal(pre, post)
    m.close()


@pytest.mark.parametrize("dt,scheme,act", [(4, 2, 1), (16, 3, 0), (5, 0, 2)])
def test_segment_dense_proxy(gpu, oracle, dt, scheme, act):
    """welvet_model_dense_proxy (dense.cpp:141-191): kind 0 is the linear
    input gradient (act' = 1), kind 1 dW with act' at the given pre, at zeros
    without one; a gradient of another length is remapped by range means."""
    rng = np.random.default_rng(60 + dt)
    W = (rng.standard_normal((48, 80)) / 9).astype(np.float32)
    # a Stack whose single child is the Dense itself (not a NestedStack)
    w = pw.Wire()
    w.u32(0x314E4D57)
    w.i32(0, 1, 1, 1, 1, 1)
    pw.dense_child(w, 80, 48, act, dt, W)
    pw.empty_controls(w)
    pw.empty_controls(w)
    w.i32(1)
    pw.store_payload(w, dt, 48, 80, oracle.pack(dt, W))
    m = pw.ModelSession(w.bytes(), scheme=scheme)
    x = rng.standard_normal((5, 80)).astype(np.float32)
    gy = rng.standard_normal((5, 48)).astype(np.float32)
    pre, _, dx_lin, _, _, _ = pw.dense_normalbp(5, 80, 48, -1, dt, scheme, W, x, gy)
    gx = m.dense_proxy(0, x, gy)
    assert gx.shape == (5, 80) and np.array_equal(gx, dx_lin)
    pre_a, _, _, dw_a, _, _ = pw.dense_normalbp(5, 80, 48, act, dt, scheme, W, x, gy)
    assert np.array_equal(m.dense_proxy(1, x, gy, pre_a), dw_a)
    native, rs, blk = oracle.quantize(dt, scheme, 48, 80, W)
    Wd = oracle.dequant(dt, scheme, 48, 80, native, rs, blk)
    _, _, dw_z = oracle.backward(Wd, gy, np.zeros((5, 48), np.float32), x, act)
    got = m.dense_proxy(1, x, gy)
    if act in (0, 5, 6, -1):
        assert np.array_equal(got, dw_z)
    else:
        assert rel_l2(got, dw_z) <= 1e-6
    # a gradient twice as long: each value the mean of a pair (f64, then f32)
    g2 = rng.standard_normal(2 * 5 * 48).astype(np.float32)
    mean = ((g2[0::2].astype(np.float64) + g2[1::2].astype(np.float64)) / 2).astype(np.float32)
    assert np.array_equal(m.dense_proxy(0, x, g2.reshape(10, 48)), m.dense_proxy(0, x, mean.reshape(5, 48)))
    m.close()


def _mixed_stack(oracle, rng, scheme):
    """Stack: Dense 96 -> 128 (ReLU, E4M3) | SwiGLU 128 / 192 (FP4) | Dense
    128 -> 80 (SiLU, E5M2), as one NestedStack child."""
    W1 = (rng.standard_normal((128, 96)) / np.sqrt(96)).astype(np.float32)
    G = (rng.standard_normal((192, 128)) / np.sqrt(128)).astype(np.float32)
    U = (rng.standard_normal((192, 128)) / np.sqrt(128)).astype(np.float32)
    D = (rng.standard_normal((128, 192)) / np.sqrt(192)).astype(np.float32)
    W3 = (rng.standard_normal((80, 128)) / np.sqrt(128)).astype(np.float32)
    w = pw.Wire()
    w.u32(0x314E4D57)
    w.i32(0, 1, 1, 1, 1, 1)
    w.i32(19, 3)
    pw.dense_child(w, 96, 128, 0, 4, W1)
    pw.swiglu_child(w, 128, 192, 16, G, U, D)
    pw.dense_child(w, 128, 80, 1, 5, W3)
    for _ in range(5):  # the stack, its child and the child's three ops
        pw.empty_controls(w)
    stores = [(4, W1), (16, G), (16, U), (16, D), (5, W3)]
    w.i32(len(stores))
    for dt, W in stores:
        pw.store_payload(w, dt, W.shape[0], W.shape[1], oracle.pack(dt, W))
    return pw.ModelSession(w.bytes(), scheme=scheme), (W1, G, U, D, W3), stores


@pytest.mark.parametrize("scheme,batch", [(0, 2), (3, 40)])
def test_segment_training_through_swiglu(gpu, oracle, scheme, batch):
    """A Stack mixing Dense and SwiGLU: welvet_model_backward gives the bits
    of the NormalBP leaves run by hand in reverse (dW: Dense, then Gate | Up |
    Down, then Dense), and SGD re-quantizes all five stores as the oracle."""
    rng = np.random.default_rng(70 + batch)
    m, (W1, G, U, D, W3), stores = _mixed_stack(oracle, rng, scheme)
    x = rng.standard_normal((batch, 96)).astype(np.float32)
    gy = rng.standard_normal((batch, 80)).astype(np.float32)
    gx, dw = m.backward(x, gy)
    _, a1 = pw.dense_forward(batch, 96, 128, 0, 4, scheme, W1, x)
    _, a2, _, _, _, _ = pw.swiglu_normalbp(batch, 1, 128, 192, 16, scheme, G, U, D, a1,
                                           np.zeros((batch, 128), np.float32))
    _, _, g3, dw3, _, _ = pw.dense_normalbp(batch, 128, 80, 1, 5, scheme, W3, a2, gy)
    _, _, g2, dw2, _, _ = pw.swiglu_normalbp(batch, 1, 128, 192, 16, scheme, G, U, D, a1, g3)
    _, _, g1, dw1, _, _ = pw.dense_normalbp(batch, 96, 128, 0, 4, scheme, W1, x, g2)
    assert np.array_equal(gx, g1)
    assert np.array_equal(dw.ravel(), np.concatenate([dw1.ravel(), dw2, dw3.ravel()]))
    lr = 0.1
    m.apply_sgd(dw, lr)
    off = 0
    for (dt, W), (sdt, rows, cols, _, native) in zip(stores, parse_nws1(m.export())):
        nat, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
        Wq = oracle.dequant(dt, scheme, rows, cols, nat, rs, blk)
        nxt = oracle.sgd(Wq, dw.ravel()[off:off + W.size].reshape(W.shape), lr)
        nat2, _, _ = oracle.quantize(dt, scheme, rows, cols, nxt)
        assert sdt == dt and np.array_equal(native, nat2), (dt, rows, cols)
        off += W.size
    m.close()


def scaled_stack(layers, stores):
    """Stack root, one NestedStack of Dense children; stores: per layer
    (dtype, scheme, native, scale, row_scale, blk_exp)."""
    w = pw.Wire()
    w.u32(0x314E4D57)
    w.i32(0, 1, 1, 1, 1, 1)
    w.i32(19, len(layers))
    for dt, W, act in layers:
        pw.dense_child(w, W.shape[1], W.shape[0], act, dt, np.zeros_like(W))
    pw.empty_controls(w)
    pw.empty_controls(w)
    for _ in layers:
        pw.empty_controls(w)
    w.i32(len(layers))
    for (dt, W, _), (sdt, scheme, native, scale, rs, blk) in zip(layers, stores):
        pw.store_payload(w, sdt, W.shape[0], W.shape[1], native, scale=scale, scheme=scheme,
                         row_scale=rs, blk_exp=blk)
    return w.bytes()


def test_scaled_store_payloads_mount_and_export(gpu, oracle):
    """Scaled stores in the WMN1 payload (the C5 cell mix: E4M3 per-row, FP4
    E8M0/32, E4M3 per-row) mount as stored, forward as the oracle chain of
    the same codes and scales, and export to NWS1 byte for byte."""
    rng = np.random.default_rng(21)
    dims = [300, 256, 192, 130]
    mix = [(4, 2), (16, 3), (4, 2)]
    layers, stores, want_chain = [], [], []
    for i, (dt, sc) in enumerate(mix):
        W = (rng.standard_normal((dims[i + 1], dims[i])) / np.sqrt(dims[i])).astype(np.float32)
        native, rs, blk = oracle.quantize(dt, sc, dims[i + 1], dims[i], W)
        layers.append((dt, W, -1))
        stores.append((dt, sc, native, 1.0, rs, blk))
        want_chain.append((dt, sc, W))
    for batch in (1, 3, 40):
        x = rng.standard_normal((batch, dims[0])).astype(np.float32)
        m = pw.ModelSession(scaled_stack(layers, stores))
        y = m.forward(x)
        cur = x
        for dt, sc, W in want_chain:
            native, rs, blk = oracle.quantize(dt, sc, W.shape[0], W.shape[1], W)
            _, cur = oracle.dense(oracle.dequant(dt, sc, W.shape[0], W.shape[1], native, rs, blk), cur)
        assert rel_l2(y, cur) <= tol(batch, chain=3)
        snap, extras = pw.parse_snapshot(m.export())
        m.close()
        assert extras == 0 and len(snap) == 3
        for (sdt, scheme, native, _, rs, blk), got in zip(stores, snap):
            dt, gsc, rows, cols, scale, f, gnat, bias = got
            assert (dt, gsc) == (sdt, scheme) and np.array_equal(gnat, native) and bias.size == 0
            if scheme == 2:
                assert np.array_equal(f, rs)
            else:
                e = np.frexp(f.astype(np.float64))[1] - 1  # f = 2^e exactly
                assert np.array_equal(np.ldexp(1.0, e), f.astype(np.float64))
                assert np.array_equal(e + 127, blk.astype(np.int64))


@pytest.mark.parametrize("scheme", [1, 2, 3])
def test_requantized_model_export_mounts_back_identically(gpu, oracle, scheme):
    """A model re-quantized at mount (welvet_model_mount_q) exports its scaled
    stores; a descriptor built from that snapshot mounts them as stored and
    gives the same outputs bit for bit."""
    rng = np.random.default_rng(30 + scheme)
    layers = [(dt, (rng.standard_normal((96, 96)) / 10).astype(np.float32), act)
              for dt, act in ((4, -1), (16, 0), (5, -1))]
    x = rng.standard_normal((24, 96)).astype(np.float32)
    m = pw.ModelSession(build_stack([layers]), scheme=scheme)
    y = m.forward(x)
    snap, _ = pw.parse_snapshot(m.export())
    m.close()
    stores = []
    for dt, sc, rows, cols, scale, f, native, _ in snap:
        assert sc == scheme
        blk = None
        if sc == 3:
            blk = (np.frexp(f.astype(np.float64))[1] - 1 + 127).astype(np.uint8)
        stores.append((dt, sc, native, scale, f if sc == 2 else None, blk))
    m2 = pw.ModelSession(scaled_stack(layers, stores))
    assert np.array_equal(m2.forward(x), y)
    snap2, _ = pw.parse_snapshot(m2.export())
    m2.close()
    for a, b in zip(snap, snap2):
        assert a[:5] == b[:5] and all(np.array_equal(u, v) for u, v in zip(a[5:], b[5:]))


def mha_child(w, seq, d, heads, kv_heads, head_dim, msl, mask, pos, dtype, Q, K, V, O):
    """MHA child (child_wire.hpp:153-192): dims, kinds, dtype, then Q, K, V, O."""
    w.i32(7, seq, d, heads, kv_heads, head_dim, msl, mask, pos, dtype)
    w.f32(np.concatenate([np.ravel(Q), np.ravel(K), np.ravel(V), np.ravel(O)]))


@pytest.mark.parametrize("B,S,d,H,KVH,msl,mask,pos,lead", [
    (2, 48, 128, 4, 2, 64, 1, 1, False),   # causal, RoPE, GQA, [B, S, d] input
    (1, 40, 64, 4, 4, 40, 2, 0, True),     # bidirectional, no positions, after a Dense child
])
def test_mha_child_matches_sessions(gpu, oracle, B, S, d, H, KVH, msl, mask, pos, lead):
    """A Stack whose ops are (a Dense child and) an MHA child, E5M2 stores as
    the reference's FormatNone payloads, against the same layers run as a
    Dense session and an MHA session (each tested against the oracle on its
    own): the model wires the child's dims, kinds, weights and stores to the
    same kernels, so the outputs agree bit for bit."""
    rng = np.random.default_rng(B * 100 + S)
    hd = d // H
    Q = (rng.standard_normal((H * hd, d)) / np.sqrt(d)).astype(np.float32)
    K = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    V = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    O = (rng.standard_normal((d, H * hd)) / np.sqrt(H * hd)).astype(np.float32)
    W1 = (rng.standard_normal((d, d)) / np.sqrt(d)).astype(np.float32)
    w = pw.Wire()
    w.u32(0x314E4D57)
    w.i32(0, 1, 1, 1, 1, 1)
    w.i32(19, 2 if lead else 1)
    if lead:
        pw.dense_child(w, d, d, 0, 4, W1)
    mha_child(w, S, d, H, KVH, 0, msl, mask, pos, 5, Q, K, V, O)
    for _ in range(3 + (1 if lead else 0)):  # the stack, its child and its ops
        pw.empty_controls(w)
    stores = ([(4, W1)] if lead else []) + [(5, Q), (5, K), (5, V), (5, O)]
    w.i32(len(stores))
    for dt, Wm in stores:
        pw.store_payload(w, dt, Wm.shape[0], Wm.shape[1], oracle.pack(dt, Wm))
    m = pw.ModelSession(w.bytes())
    x = rng.standard_normal((B, S, d) if not lead else (S, d)).astype(np.float32)
    y = m.forward(x)
    m.close()
    cur = x.reshape(B * S, d)
    if lead:
        s = pw.DenseSession(B * S, d, d, 0, 4, 0, W1)
        _, cur = s.execute(cur)
        s.close()
    sess = pw.MHASession(B, S, d, H, KVH, 0, msl, mask, pos, 5, 0, Q, K, V, O)
    _, want = sess.execute(cur)
    sess.close()
    assert y.shape == ((B, S, d) if not lead else (1, S, d))
    assert np.array_equal(y.reshape(B * S, d), want)
