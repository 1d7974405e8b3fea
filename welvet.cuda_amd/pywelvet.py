"""Python binding of libwelvet.so (the C ABI in include/welvet_c.h).

Thin ctypes layer used by the tests, the smoke check and the benchmark:
  * `lib()` loads the in-tree libwelvet.so (built by welvet.cuda_amd/Makefile)
    and declares every entry point's signature;
  * `Hip` reaches the HIP runtime that libwelvet.so itself links, for device
    buffers, streams and events (no second runtime is loaded);
  * `normal()` is the seeded synthetic-data generator (splitmix64 +
    Box-Muller in f64), so inputs are identical across runs and machines.
No computation happens here: every numeric result comes from the library.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libwelvet.so")

E4M3, E5M2, FP4 = 4, 5, 16
SCHEME_REF, SCHEME_TENSOR, SCHEME_ROW, SCHEME_BLOCK32 = 0, 1, 2, 3
LINEAR, RELU, SILU, GELU, TANH, SIGMOID, LEAKY, RELU2 = -1, 0, 1, 2, 3, 4, 5, 6


class Status(ctypes.Structure):
    _fields_ = [("code", ctypes.c_int32), ("message", ctypes.c_char * 256)]


class Blob(ctypes.Structure):
    _fields_ = [("data", ctypes.POINTER(ctypes.c_uint8)), ("size", ctypes.c_size_t)]


class WelvetError(RuntimeError):
    def __init__(self, status):
        self.code = status.code
        super().__init__(f"welvet status {status.code}: {status.message.decode(errors='replace')}")


_LIB = None
OUT_OF_PATH = (
    "welvet_model_train_credit", "welvet_model_train_mse", "welvet_model_sync",
    "welvet_rmsnorm_forward_f32", "welvet_rmsnorm_normalbp_f32",
    "welvet_layernorm_forward_f32", "welvet_layernorm_normalbp_f32", "welvet_softmax_forward_f32",
    "welvet_softmax_normalbp_f32", "welvet_embedding_forward_f32",
    "welvet_embedding_normalbp_f32", "welvet_mha_normalbp_f32", "welvet_cnn1_forward_f32",
    "welvet_cnn1_normalbp_f32", "welvet_cnn2_forward_f32", "welvet_cnn2_normalbp_f32",
    "welvet_cnn3_forward_f32", "welvet_cnn3_normalbp_f32", "welvet_convt1_forward_f32",
    "welvet_convt1_normalbp_f32", "welvet_convt2_forward_f32", "welvet_convt2_normalbp_f32",
    "welvet_convt3_forward_f32", "welvet_convt3_normalbp_f32", "welvet_rnn_forward_f32",
    "welvet_rnn_normalbp_f32", "welvet_lstm_forward_f32", "welvet_lstm_normalbp_f32",
    "welvet_sequential_forward_f32", "welvet_sequential_normalbp_f32",
    "welvet_residual_forward_f32", "welvet_residual_normalbp_f32", "welvet_stack_normalbp_f32",
    "welvet_mamba_normalbp_f32", "welvet_metacognition_normalbp_f32", "welvet_gdn_normalbp_f32",
    "welvet_kmeans_normalbp_f32", "welvet_parallel_normalbp_f32", "welvet_mamba_forward_f32",
    "welvet_metacognition_forward_f32", "welvet_gdn_forward_f32", "welvet_kmeans_forward_f32",
    "welvet_parallel_forward_f32",
)
_i32, _u32, _sz, _f64 = ctypes.c_int32, ctypes.c_uint32, ctypes.c_size_t, ctypes.c_double
_vp = ctypes.c_void_p
_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i64p = ctypes.POINTER(ctypes.c_int64)


def _sig(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args


def lib():
    """Loads the in-tree library (raises if it was not built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -f welvet.cuda_amd/Makefile`")
    L = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    _sig(L, "welvet_version", ctypes.c_char_p, [])
    _sig(L, "welvet_runtime_identity", ctypes.c_char_p, [])
    _sig(L, "welvet_cuda_init", Status, [])
    _sig(L, "welvet_cuda_available", _i32, [])
    _sig(L, "welvet_gaps_count", _i32, [])
    _sig(L, "welvet_gaps_done", _i32, [])
    _sig(L, "welvet_dense_forward_f32", Status,
         [_i32, _i32, _i32, _i32, _i32, _i32, _fp, _dp, _sz, _fp, _fp, _fp])
    _sig(L, "welvet_dense_normalbp_f32", Status,
         [_i32, _i32, _i32, _i32, _i32, _i32, _fp, _dp, _sz, _fp, _fp, _i32, _f64, _fp, _fp, _fp,
          _fp, _fp, _dp])
    _sig(L, "welvet_swiglu_normalbp_f32", Status,
         [_i32] * 6 + [_fp] * 5 + [_i32, _f64] + [_fp] * 5 + [_dp])
    _sig(L, "welvet_dense_mount", Status,
         [_i32, _i32, _i32, _i32, _i32, _fp, _dp, _sz, ctypes.POINTER(_vp)])
    _sig(L, "welvet_dense_mount_q", Status,
         [_i32, _i32, _i32, _i32, _i32, _i32, _fp, _dp, _sz, ctypes.POINTER(_vp)])
    _sig(L, "welvet_dense_execute", Status, [_vp, _fp, _fp, _fp])
    _sig(L, "welvet_dense_execute_device", Status, [_vp, _vp, _vp, _vp, _vp])
    _sig(L, "welvet_dense_execute_noalloc", Status, [_vp, _i32, _vp, _vp, _vp, _vp])
    _sig(L, "welvet_dense_backward_device", Status,
         [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp])
    _sig(L, "welvet_dense_export_store", Status,
         [_vp, _u8p, _sz, ctypes.POINTER(_sz), _fp, _u8p, _fp])
    _sig(L, "welvet_dense_release", None, [_vp])
    _sig(L, "welvet_dense_mount_format", Status,
         [_i32, _i32, _i32, _i32, _i32, _fp, _u8p, _sz, _dp, _sz, ctypes.POINTER(_vp)])
    _sig(L, "welvet_dense_export_blocks", Status, [_vp, _u8p, _sz, ctypes.POINTER(_sz)])
    _sig(L, "welvet_dense_export_f32", Status, [_vp, _fp])
    _sig(L, "welvet_dense_group_mount", Status,
         [ctypes.POINTER(_vp), _i32, ctypes.POINTER(_vp), ctypes.POINTER(_vp),
          ctypes.POINTER(_vp), ctypes.POINTER(_vp)])
    _sig(L, "welvet_dense_group_execute", Status, [_vp, _vp])
    _sig(L, "welvet_dense_group_release", None, [_vp])
    _sig(L, "welvet_dense_chain_mount", Status, [_vp, ctypes.c_int32, _vp])
    _sig(L, "welvet_dense_chain_mount_ex", Status, [_vp, ctypes.c_int32, ctypes.c_int32, _vp])
    _sig(L, "welvet_dense_chain_execute", Status, [_vp, _vp])
    _sig(L, "welvet_dense_chain_release", None, [_vp])
    _sig(L, "welvet_swiglu_forward_f32", Status,
         [_i32, _i32, _i32, _i32, _i32, _i32, _fp, _fp, _fp, _fp, _fp, _fp])
    _sig(L, "welvet_swiglu_mount", Status,
         [_i32, _i32, _i32, _i32, _i32, _i32, _fp, _fp, _fp, ctypes.POINTER(_vp)])
    _sig(L, "welvet_swiglu_execute", Status, [_vp, _fp, _fp, _fp])
    _sig(L, "welvet_swiglu_execute_device", Status, [_vp, _vp, _vp, _vp, _vp])
    _sig(L, "welvet_swiglu_release", None, [_vp])
    _sig(L, "welvet_mha_forward_f32", Status,
         [_i32] * 11 + [_fp, _fp, _fp, _fp, _fp, _fp, _fp])
    _sig(L, "welvet_mha_mount", Status, [_i32] * 11 + [_fp, _fp, _fp, _fp, ctypes.POINTER(_vp)])
    _sig(L, "welvet_mha_execute", Status, [_vp, _fp, _fp, _fp])
    _sig(L, "welvet_mha_execute_device", Status, [_vp, _vp, _vp, _vp, _vp])
    _sig(L, "welvet_mha_release", None, [_vp])
    _sig(L, "welvet_model_abi_version", _i32, [])
    _sig(L, "welvet_model_mount", Status, [_u8p, _sz, ctypes.POINTER(_vp)])
    _sig(L, "welvet_model_mount_q", Status, [_u8p, _sz, _i32, ctypes.POINTER(_vp)])
    _sig(L, "welvet_model_forward", Status, [_vp, _u8p, _sz, ctypes.POINTER(Blob)])
    _sig(L, "welvet_model_forward_device", Status, [_vp, _vp, _i32, _i32, _vp, _i32, _vp])
    _sig(L, "welvet_model_export_weights", Status, [_vp, ctypes.POINTER(Blob)])
    _sig(L, "welvet_model_backward", Status, [_vp, _u8p, _sz, ctypes.POINTER(Blob)])
    _sig(L, "welvet_model_apply_sgd", Status, [_vp, _f64, _u8p, _sz])
    _sig(L, "welvet_model_forward_pair", Status, [_vp, _u8p, _sz, ctypes.POINTER(Blob)])
    _sig(L, "welvet_model_dense_proxy", Status, [_vp, _i32, _u8p, _sz, ctypes.POINTER(Blob)])
    _sig(L, "welvet_model_release", None, [_vp])
    _sig(L, "welvet_cuda_blob_free", None, [ctypes.POINTER(Blob)])
    _sig(L, "welvet_codec_sweep", Status, [_i32, _u32, _u32, _i64p])
    _sig(L, "welvet_read_probe", Status, [_vp, _sz, _vp, _sz, _vp])
    _sig(L, "welvet_read_probe_words", _sz, [_sz])
    _sig(L, "welvet_fetch_probe", Status, [_vp, _sz, _i32, _i32, _vp, _sz, _vp])
    _sig(L, "welvet_mfma_probe", Status, [_i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp])
    _sig(L, "welvet_clock_stamp", Status, [_vp, _vp])
    _sig(L, "welvet_clock_rate_khz", ctypes.c_int64, [])
    _sig(L, "welvet_seqmix_kind_name", Status, [_i32, ctypes.c_char_p, _i32])
    for n in ("welvet_seqmix_mha_kind", "welvet_seqmix_mamba_kind", "welvet_seqmix_gdn_kind"):
        _sig(L, n, _i32, [])
    # Entry points outside the quantized Dense path return welvet_status by
    # value (code 3); ctypes must know the struct return to pass its slot.
    for n in OUT_OF_PATH:
        getattr(L, n).restype = Status
    _LIB = L
    return L


def check(st):
    if st.code != 0:
        raise WelvetError(st)
    return st


def fptr(a):
    return a.ctypes.data_as(_fp) if a is not None else None


def dptr(a):
    return a.ctypes.data_as(_dp) if a is not None else None


# --------------------------------------------------------------------------
def normal(seed, n, std=1.0):
    """n samples of N(0, std^2) as float32: splitmix64 stream from `seed`,
    uniforms ((z >> 11) + 0.5) * 2^-53, Box-Muller pairs (cos, sin)."""
    m = (n + 1) // 2
    with np.errstate(over="ignore"):
        k = np.arange(1, 2 * m + 1, dtype=np.uint64)
        z = np.uint64(seed) + k * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    u = ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    out = np.empty(2 * m, dtype=np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    return (out[:n] * std).astype(np.float32)


def seed_for(config, cell=0):
    return 0x5EED0000 + config * 1000 + cell


# --------------------------------------------------------------------------
class Hip:
    """Device buffers, streams and events from the HIP runtime libwelvet links."""

    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        lib()
        h = ctypes.CDLL("libamdhip64.so.7")
        _sig(h, "hipMalloc", ctypes.c_int, [ctypes.POINTER(_vp), _sz])
        _sig(h, "hipFree", ctypes.c_int, [_vp])
        _sig(h, "hipMemcpy", ctypes.c_int, [_vp, _vp, _sz, ctypes.c_int])
        _sig(h, "hipMemset", ctypes.c_int, [_vp, ctypes.c_int, _sz])
        _sig(h, "hipMemcpyAsync", ctypes.c_int, [_vp, _vp, _sz, ctypes.c_int, _vp])
        _sig(h, "hipDeviceSynchronize", ctypes.c_int, [])
        _sig(h, "hipStreamCreate", ctypes.c_int, [ctypes.POINTER(_vp)])
        _sig(h, "hipStreamDestroy", ctypes.c_int, [_vp])
        _sig(h, "hipStreamSynchronize", ctypes.c_int, [_vp])
        _sig(h, "hipEventCreate", ctypes.c_int, [ctypes.POINTER(_vp)])
        _sig(h, "hipEventDestroy", ctypes.c_int, [_vp])
        _sig(h, "hipEventRecord", ctypes.c_int, [_vp, _vp])
        _sig(h, "hipEventSynchronize", ctypes.c_int, [_vp])
        _sig(h, "hipEventElapsedTime", ctypes.c_int, [_fp, _vp, _vp])
        _sig(h, "hipGetErrorString", ctypes.c_char_p, [ctypes.c_int])
        _sig(h, "hipStreamBeginCapture", ctypes.c_int, [_vp, ctypes.c_int])
        _sig(h, "hipStreamEndCapture", ctypes.c_int, [_vp, ctypes.POINTER(_vp)])
        _sig(h, "hipGraphInstantiate", ctypes.c_int,
             [ctypes.POINTER(_vp), _vp, _vp, ctypes.c_char_p, _sz])
        _sig(h, "hipGraphLaunch", ctypes.c_int, [_vp, _vp])
        _sig(h, "hipGraphExecDestroy", ctypes.c_int, [_vp])
        _sig(h, "hipGraphDestroy", ctypes.c_int, [_vp])
        _sig(h, "hipHostMalloc", ctypes.c_int, [ctypes.POINTER(_vp), _sz, ctypes.c_uint])
        _sig(h, "hipHostFree", ctypes.c_int, [_vp])
        self.h = h
        self._stage = None

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.h.hipGetErrorString(rc).decode()}")

    def malloc(self, nbytes):
        p = _vp()
        self._ok(self.h.hipMalloc(ctypes.byref(p), max(int(nbytes), 16)), "hipMalloc")
        return p.value

    def free(self, p):
        if p:
            self._ok(self.h.hipFree(_vp(p)), "hipFree")

    STAGE = 8 << 20

    def _staging(self):
        """Pinned host buffer for host <-> device copies: the runtime is never
        handed pageable memory to pin in place."""
        if self._stage is None:
            b = _vp()
            self._ok(self.h.hipHostMalloc(ctypes.byref(b), self.STAGE, 0), "hipHostMalloc")
            self._stage = b.value
        return self._stage

    def _h2d(self, dev, host_addr, nbytes):
        st = self._staging()
        for off in range(0, nbytes, self.STAGE):
            n = min(self.STAGE, nbytes - off)
            ctypes.memmove(st, host_addr + off, n)
            self._ok(self.h.hipMemcpy(_vp(dev + off), _vp(st), n, self.H2D), "H2D")

    def _d2h(self, host_addr, dev, nbytes):
        st = self._staging()
        for off in range(0, nbytes, self.STAGE):
            n = min(self.STAGE, nbytes - off)
            self._ok(self.h.hipMemcpy(_vp(st), _vp(dev + off), n, self.D2H), "D2H")
            ctypes.memmove(host_addr + off, st, n)

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.malloc(arr.nbytes)
        self._h2d(p, arr.ctypes.data, arr.nbytes)
        return p

    def copy_in(self, p, arr):
        """Host array into an existing device buffer; returns once it has landed."""
        arr = np.ascontiguousarray(arr)
        self._h2d(p, arr.ctypes.data, arr.nbytes)
        self.sync()

    def download(self, p, shape, dtype=np.float32):
        out = np.empty(shape, dtype=dtype)
        self._d2h(out.ctypes.data, p, out.nbytes)
        return out

    def copy_async(self, dst, src, nbytes, stream):
        """Device-to-device copy queued on `stream`."""
        self._ok(self.h.hipMemcpyAsync(_vp(dst), _vp(src), nbytes, self.D2D, _vp(stream)),
                 "hipMemcpyAsync")

    def memset(self, p, value, nbytes):
        self._ok(self.h.hipMemset(_vp(p), value, nbytes), "hipMemset")

    def sync(self):
        self._ok(self.h.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream(self):
        s = _vp()
        self._ok(self.h.hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        return s.value

    def stream_sync(self, s):
        self._ok(self.h.hipStreamSynchronize(_vp(s)), "hipStreamSynchronize")

    def event(self):
        e = _vp()
        self._ok(self.h.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e.value

    def record(self, e, s):
        self._ok(self.h.hipEventRecord(_vp(e), _vp(s)), "hipEventRecord")

    def capture(self, stream, enqueue):
        """Records what enqueue() queues on `stream` into an instantiated graph."""
        self._ok(self.h.hipStreamBeginCapture(_vp(stream), 2), "hipStreamBeginCapture")
        try:
            enqueue()
        finally:
            g = _vp()
            rc = self.h.hipStreamEndCapture(_vp(stream), ctypes.byref(g))
        self._ok(rc, "hipStreamEndCapture")
        ex = _vp()
        self._ok(self.h.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        self._ok(self.h.hipGraphDestroy(g), "hipGraphDestroy")
        return ex.value

    def launch(self, graph_exec, stream):
        self._ok(self.h.hipGraphLaunch(_vp(graph_exec), _vp(stream)), "hipGraphLaunch")

    def graph_free(self, graph_exec):
        self._ok(self.h.hipGraphExecDestroy(_vp(graph_exec)), "hipGraphExecDestroy")

    def elapsed_ms(self, a, b):
        self._ok(self.h.hipEventSynchronize(_vp(b)), "hipEventSynchronize")
        t = ctypes.c_float()
        self._ok(self.h.hipEventElapsedTime(ctypes.byref(t), _vp(a), _vp(b)), "hipEventElapsedTime")
        return t.value


# --------------------------------------------------------------------------
CHAIN_INNER_NOT_KEPT = 1


class DenseChain:
    """Groups run in order, each reading the previous group's outputs.
    keep_inner=False: groups whose epilogue writes the next group's split do
    not write their own outputs (WELVET_CHAIN_INNER_NOT_KEPT)."""

    def __init__(self, groups, keep_inner=True):
        n = len(groups)
        self._groups = list(groups)  # the groups must outlive the chain
        h = _vp()
        arr = (_vp * n)(*[g.h for g in groups])
        if keep_inner:
            check(lib().welvet_dense_chain_mount(arr, n, ctypes.byref(h)))
        else:
            check(lib().welvet_dense_chain_mount_ex(arr, n, CHAIN_INNER_NOT_KEPT, ctypes.byref(h)))
        self.h = h

    def execute(self, stream=None):
        check(lib().welvet_dense_chain_execute(self.h, _vp(stream) if stream else None))

    def close(self):
        if self.h:
            lib().welvet_dense_chain_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DenseGroup:
    """Grouped execution of same-shape Dense sessions over fixed device buffers."""

    def __init__(self, sessions, xs, pres, posts):
        n = len(sessions)
        arr = lambda vals: (_vp * n)(*[_vp(v) for v in vals])
        self._sessions = list(sessions)  # the sessions must outlive the group
        h = _vp()
        check(lib().welvet_dense_group_mount(arr([s.h.value for s in sessions]), n, arr(xs),
                                             arr(pres), arr(posts), ctypes.byref(h)))
        self.h = h

    def execute(self, stream=None):
        check(lib().welvet_dense_group_execute(self.h, _vp(stream) if stream else None))

    def close(self):
        if self.h:
            lib().welvet_dense_group_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DenseSession:
    """welvet_dense_mount_q / execute / execute_device / export_store / release."""

    def __init__(self, batch, in_dim, out_dim, act, dtype, scheme, W, bias=None):
        L = lib()
        self.batch, self.in_dim, self.out_dim = batch, in_dim, out_dim
        W = np.ascontiguousarray(W, dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float64)
        h = _vp()
        check(L.welvet_dense_mount_q(batch, in_dim, out_dim, act, dtype, scheme, fptr(W), dptr(b),
                                     0 if b is None else b.size, ctypes.byref(h)))
        self.h = h

    def execute(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        pre = np.empty((self.batch, self.out_dim), np.float32)
        post = np.empty_like(pre)
        check(lib().welvet_dense_execute(self.h, fptr(x), fptr(pre), fptr(post)))
        return pre, post

    def execute_device(self, x, pre, post, stream=None):
        check(lib().welvet_dense_execute_device(self.h, _vp(x), _vp(pre), _vp(post),
                                                _vp(stream) if stream else None))

    def execute_noalloc(self, rows, x, pre, post, stream=None):
        check(lib().welvet_dense_execute_noalloc(self.h, rows, _vp(x), _vp(pre), _vp(post),
                                                 _vp(stream) if stream else None))

    def backward_device(self, x, pre, post, g, use_target, dpre, dx, dw, loss_part=None,
                        stream=None):
        check(lib().welvet_dense_backward_device(self.h, _vp(x), _vp(pre), _vp(post), _vp(g),
                                                 1 if use_target else 0, _vp(dpre), _vp(dx),
                                                 _vp(dw), _vp(loss_part) if loss_part else None,
                                                 _vp(stream) if stream else None))

    def export_store(self, dtype):
        n = self.in_dim * self.out_dim
        cap = n if dtype != FP4 else (n + 1) // 2
        native = np.zeros(cap, np.uint8)
        nlen = _sz()
        rs = np.zeros(self.out_dim, np.float32)
        blk = np.zeros(self.out_dim * ((self.in_dim + 31) // 32), np.uint8)
        ts = ctypes.c_float()
        check(lib().welvet_dense_export_store(self.h, native.ctypes.data_as(_u8p), cap,
                                              ctypes.byref(nlen), fptr(rs),
                                              blk.ctypes.data_as(_u8p), ctypes.byref(ts)))
        return native[: nlen.value], rs, blk, ts.value

    def export_f32(self):
        W = np.zeros((self.out_dim, self.in_dim), np.float32)
        check(lib().welvet_dense_export_f32(self.h, fptr(W)))
        return W

    def close(self):
        if self.h:
            lib().welvet_dense_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# packed block formats (QuantFormat ids of welvet_dense_mount_format)
Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 1, 2, 3, 4, 5, 6, 7, 8, 9, 10
IQ4_NL, IQ4_XS = 16, 17


class FormatDenseSession(DenseSession):
    """welvet_dense_mount_format: a Dense session over a packed block format,
    from fp32 weights W (quantized on the device) or from packed blocks."""

    def __init__(self, batch, in_dim, out_dim, act, fmt, W=None, blocks=None, bias=None):
        L = lib()
        self.batch, self.in_dim, self.out_dim, self.fmt = batch, in_dim, out_dim, fmt
        self.h = None
        Wc = None if W is None else np.ascontiguousarray(W, dtype=np.float32)
        bc = None if blocks is None else np.ascontiguousarray(blocks, dtype=np.uint8)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float64)
        h = _vp()
        check(L.welvet_dense_mount_format(
            batch, in_dim, out_dim, act, fmt, fptr(Wc) if Wc is not None else None,
            bc.ctypes.data_as(_u8p) if bc is not None else None, 0 if bc is None else bc.size,
            dptr(b), 0 if b is None else b.size, ctypes.byref(h)))
        self.h = h

    def export_blocks(self):
        n = _sz()
        check(lib().welvet_dense_export_blocks(self.h, None, 0, ctypes.byref(n)))
        out = np.zeros(n.value, np.uint8)
        check(lib().welvet_dense_export_blocks(self.h, out.ctypes.data_as(_u8p), out.size,
                                               ctypes.byref(n)))
        return out


class SwiGLUSession:
    def __init__(self, batch, seq, in_dim, inter, dtype, scheme, G, U, D):
        L = lib()
        self.rows, self.in_dim, self.inter = batch * seq, in_dim, inter
        self._keep = [np.ascontiguousarray(a, dtype=np.float32) for a in (G, U, D)]
        h = _vp()
        check(L.welvet_swiglu_mount(batch, seq, in_dim, inter, dtype, scheme,
                                    *[fptr(a) for a in self._keep], ctypes.byref(h)))
        self._keep = None
        self.h = h

    def execute(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        pre = np.empty((self.rows, self.inter), np.float32)
        post = np.empty((self.rows, self.in_dim), np.float32)
        check(lib().welvet_swiglu_execute(self.h, fptr(x), fptr(pre), fptr(post)))
        return pre, post

    def execute_device(self, x, pre, post, stream=None):
        check(lib().welvet_swiglu_execute_device(self.h, _vp(x), _vp(pre), _vp(post),
                                                 _vp(stream) if stream else None))

    def close(self):
        if self.h:
            lib().welvet_swiglu_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MHASession:
    def __init__(self, batch, seq, d_model, heads, kv_heads, head_dim, msl, mask, pos, dtype,
                 scheme, Q, K, V, O):
        L = lib()
        self.batch, self.seq, self.d = batch, seq, d_model
        hd = head_dim if head_dim > 0 else d_model // heads
        self.q_dim = heads * hd
        keep = [np.ascontiguousarray(a, dtype=np.float32) for a in (Q, K, V, O)]
        h = _vp()
        check(L.welvet_mha_mount(batch, seq, d_model, heads, kv_heads, head_dim, msl, mask, pos,
                                 dtype, scheme, *[fptr(a) for a in keep], ctypes.byref(h)))
        self.h = h

    def execute(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = self.batch * self.seq
        pre = np.empty((T, self.q_dim), np.float32)
        post = np.empty((T, self.d), np.float32)
        check(lib().welvet_mha_execute(self.h, fptr(x), fptr(pre), fptr(post)))
        return pre, post

    def execute_device(self, x, pre, post, stream=None):
        check(lib().welvet_mha_execute_device(self.h, _vp(x), _vp(pre), _vp(post),
                                              _vp(stream) if stream else None))

    def close(self):
        if self.h:
            lib().welvet_mha_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def dense_forward(batch, in_dim, out_dim, act, dtype, scheme, W, x, bias=None):
    """welvet_dense_forward_f32 (one shot)."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float64)
    pre = np.empty((batch, out_dim), np.float32)
    post = np.empty_like(pre)
    check(lib().welvet_dense_forward_f32(batch, in_dim, out_dim, act, dtype, scheme, fptr(W),
                                         dptr(b), 0 if b is None else b.size, fptr(x), fptr(pre),
                                         fptr(post)))
    return pre, post


def dense_normalbp(batch, in_dim, out_dim, act, dtype, scheme, W, x, grad_or_target,
                   use_target=False, lr=0.0, bias=None):
    """welvet_dense_normalbp_f32: forward, backward over the quantized weights
    and optional SGD. Returns pre, post, dX, dW, W_after, loss."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(grad_or_target, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float64)
    pre = np.empty((batch, out_dim), np.float32)
    post = np.empty_like(pre)
    dx = np.empty((batch, in_dim), np.float32)
    dw = np.empty((out_dim, in_dim), np.float32)
    wa = np.empty((out_dim, in_dim), np.float32)
    loss = np.zeros(1, np.float64)
    check(lib().welvet_dense_normalbp_f32(batch, in_dim, out_dim, act, dtype, scheme, fptr(W),
                                          dptr(b), 0 if b is None else b.size, fptr(x), fptr(g),
                                          1 if use_target else 0, float(lr), fptr(pre),
                                          fptr(post), fptr(dx), fptr(dw), fptr(wa), dptr(loss)))
    return pre, post, dx, dw, wa, float(loss[0])


def swiglu_normalbp(batch, seq, in_dim, inter, dtype, scheme, G, U, D, x, grad_or_target,
                    use_target=False, lr=0.0):
    """welvet_swiglu_normalbp_f32: pre (h), post (y), dX, dW, W_after, loss."""
    arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (G, U, D, x, grad_or_target)]
    rows = batch * seq
    pre = np.empty((rows, inter), np.float32)
    post = np.empty((rows, in_dim), np.float32)
    dx = np.empty((rows, in_dim), np.float32)
    dw = np.empty(3 * inter * in_dim, np.float32)
    wa = np.empty_like(dw)
    loss = np.zeros(1, np.float64)
    check(lib().welvet_swiglu_normalbp_f32(batch, seq, in_dim, inter, dtype, scheme,
                                           *[fptr(a) for a in arrs], 1 if use_target else 0,
                                           float(lr), fptr(pre), fptr(post), fptr(dx), fptr(dw),
                                           fptr(wa), dptr(loss)))
    return pre, post, dx, dw, wa, float(loss[0])


def codec_sweep(dtype, first_chunk=0, n_chunks=4096):
    out = np.zeros(2 * n_chunks, np.int64)
    check(lib().welvet_codec_sweep(dtype, first_chunk, n_chunks, out.ctypes.data_as(_i64p)))
    return out.reshape(n_chunks, 2)


# --------------------------------------------------------------- WMN1 -----
class Wire:
    """Little-endian writer for WMN1 descriptors and tensors
    (src/interop/model_session.cpp:101-162 layouts)."""

    def __init__(self):
        self.parts = []

    def i32(self, *v):
        self.parts.append(np.asarray(v, dtype="<i4").tobytes())

    def u32(self, *v):
        self.parts.append(np.asarray(v, dtype="<u4").tobytes())

    def f32(self, arr):
        self.parts.append(np.ascontiguousarray(arr, dtype="<f4").tobytes())

    def f64(self, arr):
        self.parts.append(np.ascontiguousarray(arr, dtype="<f8").tobytes())

    def u8(self, arr):
        self.parts.append(np.ascontiguousarray(arr, dtype=np.uint8).tobytes())

    def bytes(self):
        return b"".join(self.parts)


def dense_child(w, in_dim, out_dim, act, dtype, W, bias=None):
    w.i32(1, in_dim, out_dim, act, dtype)
    w.f32(W)
    b = np.zeros(0) if bias is None else np.asarray(bias, np.float64)
    w.u32(b.size)
    if b.size:
        w.f64(b)


def swiglu_child(w, in_dim, inter, dtype, G, U, D):
    """SwiGLU child (child_wire.hpp:95-118): dims, dtype, then Gate, Up, Down."""
    w.i32(4, in_dim, inter, dtype)
    w.f32(np.concatenate([np.ravel(G), np.ravel(U), np.ravel(D)]))


def empty_controls(w):
    # modes, branch_lrs, shadow_coef, surprise_thresh, last_loss, sync present
    w.i32(0, 0)
    w.f64([0.0, 0.0, 0.0])
    w.i32(0)


def store_payload(w, dtype, rows, cols, native, scale=1.0, bias=None, scheme=0, row_scale=None,
                  blk_exp=None):
    """One store of a WMN1 descriptor (model_session.cpp:135-162). scheme 0 is
    the reference's FormatNone store (no f32 payload); schemes 1-3 are this
    library's scaled extension: the dtype word carries the scheme in bits
    8-15, the tensor scale goes in `scale` (1), the row scales (2) or the
    E8M0 block scales as powers of two (3) in the f32 payload."""
    w.i32(dtype | (scheme << 8), rows, cols)
    w.f32([scale])
    if scheme == 2:
        f = np.asarray(row_scale, np.float32)
    elif scheme == 3:
        e = np.asarray(blk_exp, np.int64) - 127
        f = np.where(e >= -126, np.ldexp(1.0, e), 2.0 ** -127).astype(np.float32)
    else:
        f = np.zeros(0, np.float32)
    w.i32(f.size)
    if f.size:
        w.f32(f)
    w.i32(len(native))
    w.u8(native)
    b = np.zeros(0) if bias is None else np.asarray(bias, np.float64)
    w.i32(b.size)
    if b.size:
        w.f64(b)


def parse_snapshot(raw):
    """NWS1 blob -> list of stores (dtype, scheme, rows, cols, scale, f32,
    native, bias) and the extras count."""
    assert raw[:4] == b"NWS1"
    off = 4
    n = int(np.frombuffer(raw[off:off + 4], "<i4")[0])
    off += 4
    out = []
    for _ in range(n):
        tag, rows, cols = np.frombuffer(raw[off:off + 12], "<i4").tolist()
        scale = float(np.frombuffer(raw[off + 12:off + 16], "<f4")[0])
        off += 16
        nf = int(np.frombuffer(raw[off:off + 4], "<i4")[0])
        f = np.frombuffer(raw[off + 4:off + 4 + 4 * nf], "<f4").copy()
        off += 4 + 4 * nf
        nn = int(np.frombuffer(raw[off:off + 4], "<i4")[0])
        native = np.frombuffer(raw[off + 4:off + 4 + nn], np.uint8).copy()
        off += 4 + nn
        nb = int(np.frombuffer(raw[off:off + 4], "<i4")[0])
        bias = np.frombuffer(raw[off + 4:off + 4 + 8 * nb], "<f8").copy()
        off += 4 + 8 * nb
        out.append((tag & 0xFF, (tag >> 8) & 0xFF, rows, cols, scale, f, native, bias))
    extras = int(np.frombuffer(raw[off:off + 4], "<i4")[0])
    return out, extras


def tensor_bytes(x):
    w = Wire()
    w.i32(x.ndim, *x.shape)
    w.f32(x)
    return w.bytes()


class ModelSession:
    def __init__(self, descriptor, scheme=0):
        L = lib()
        buf = np.frombuffer(descriptor, dtype=np.uint8).copy()
        h = _vp()
        if scheme:
            check(L.welvet_model_mount_q(buf.ctypes.data_as(_u8p), buf.size, scheme, ctypes.byref(h)))
        else:
            check(L.welvet_model_mount(buf.ctypes.data_as(_u8p), buf.size, ctypes.byref(h)))
        self.h = h

    def forward(self, x):
        data = np.frombuffer(tensor_bytes(np.ascontiguousarray(x, np.float32)), np.uint8).copy()
        blob = Blob()
        check(lib().welvet_model_forward(self.h, data.ctypes.data_as(_u8p), data.size,
                                         ctypes.byref(blob)))
        try:
            raw = bytes(ctypes.cast(blob.data, ctypes.POINTER(ctypes.c_uint8 * blob.size)).contents)
        finally:
            lib().welvet_cuda_blob_free(ctypes.byref(blob))
        rank = int(np.frombuffer(raw[:4], "<i4")[0])
        shape = tuple(np.frombuffer(raw[4:4 + 4 * rank], "<i4").tolist())
        count = int(np.frombuffer(raw[4 + 4 * rank:8 + 4 * rank], "<i4")[0])
        data = np.frombuffer(raw[8 + 4 * rank:], "<f4")
        assert data.size == count
        return data.reshape(shape)

    @staticmethod
    def _tensors(raw, n):
        """n model-wire tensors (rank, dims, count, float32 data) from a blob."""
        out, off = [], 0
        for _ in range(n):
            rank = int(np.frombuffer(raw[off:off + 4], "<i4")[0])
            shape = tuple(np.frombuffer(raw[off + 4:off + 4 + 4 * rank], "<i4").tolist())
            off += 4 + 4 * rank
            count = int(np.frombuffer(raw[off:off + 4], "<i4")[0])
            off += 4
            out.append(np.frombuffer(raw[off:off + 4 * count], "<f4").reshape(shape).copy())
            off += 4 * count
        assert off == len(raw)
        return out

    def backward(self, x, gy):
        """welvet_model_backward: (input gradient, concatenated dW [1, n])."""
        data = np.frombuffer(tensor_bytes(np.ascontiguousarray(x, np.float32))
                             + tensor_bytes(np.ascontiguousarray(gy, np.float32)), np.uint8).copy()
        blob = Blob()
        check(lib().welvet_model_backward(self.h, data.ctypes.data_as(_u8p), data.size,
                                          ctypes.byref(blob)))
        try:
            raw = bytes(ctypes.cast(blob.data, ctypes.POINTER(ctypes.c_uint8 * blob.size)).contents)
        finally:
            lib().welvet_cuda_blob_free(ctypes.byref(blob))
        gx, dw = self._tensors(raw, 2)
        return gx, dw

    def _call_blob(self, fn, data, n, *lead):
        data = np.frombuffer(data, np.uint8).copy()
        blob = Blob()
        check(fn(self.h, *lead, data.ctypes.data_as(_u8p), data.size, ctypes.byref(blob)))
        try:
            raw = bytes(ctypes.cast(blob.data, ctypes.POINTER(ctypes.c_uint8 * blob.size)).contents)
        finally:
            lib().welvet_cuda_blob_free(ctypes.byref(blob))
        return self._tensors(raw, n)

    def forward_pair(self, x):
        """welvet_model_forward_pair: (last op's pre-activation, output)."""
        return tuple(self._call_blob(lib().welvet_model_forward_pair,
                                     tensor_bytes(np.ascontiguousarray(x, np.float32)), 2))

    def dense_proxy(self, kind, x, gy, pre=None):
        """welvet_model_dense_proxy: kind 0 linear input gradient, 1 dW."""
        w = Wire()
        data = (tensor_bytes(np.ascontiguousarray(x, np.float32))
                + tensor_bytes(np.ascontiguousarray(gy, np.float32)))
        w.i32(0 if pre is None else 1)
        data += w.bytes()
        if pre is not None:
            data += tensor_bytes(np.ascontiguousarray(pre, np.float32))
        return self._call_blob(lib().welvet_model_dense_proxy, data, 1, kind)[0]

    def apply_sgd(self, dw, lr):
        data = np.frombuffer(tensor_bytes(np.ascontiguousarray(dw, np.float32)), np.uint8).copy()
        check(lib().welvet_model_apply_sgd(self.h, float(lr), data.ctypes.data_as(_u8p), data.size))

    def forward_device(self, x, batch, width, y, y_cap, stream=None):
        check(lib().welvet_model_forward_device(self.h, _vp(x), batch, width, _vp(y), y_cap,
                                                _vp(stream) if stream else None))

    def export(self):
        blob = Blob()
        check(lib().welvet_model_export_weights(self.h, ctypes.byref(blob)))
        try:
            return bytes(ctypes.cast(blob.data, ctypes.POINTER(ctypes.c_uint8 * blob.size)).contents)
        finally:
            lib().welvet_cuda_blob_free(ctypes.byref(blob))

    def close(self):
        if self.h:
            lib().welvet_model_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
