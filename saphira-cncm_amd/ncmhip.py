"""ctypes binding of libncmhip.so, the C ABI declared in include/ncm_hip.h.

This is the host-side mirror used by the tests and the benchmark: numpy
arrays in, device buffers allocated through the library's own allocator,
every call checked through ncm_hip_last_error.  It never falls back to a
CPU path: if libncmhip.so is missing or the GPU is unusable, it raises.
"""
import ctypes
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libncmhip.so")
HEADER = os.path.join(REPO, "include", "ncm_hip.h")

ACT = {"none": 0, "silu": 1, "gelu": 2, "gelu_tanh": 3, "relu2": 4}

c_float_p = ctypes.POINTER(ctypes.c_float)
vp = ctypes.c_void_p
i64 = ctypes.c_int64
ci = ctypes.c_int
sz = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGS = {
    "ncm_hip_init": (ci, [ci]),
    "ncm_hip_set_error_mode": (None, [ci]),
    "ncm_hip_last_error": (ci, [ctypes.c_char_p, sz]),
    "ncm_hip_sync": (None, []),
    "ncm_hip_stream": (vp, []),
    "ncm_hip_malloc": (vp, [sz]),
    "ncm_hip_free": (None, [vp]),
    "ncm_hip_fail_alloc_after": (None, [ctypes.c_long]),
    "ncm_vq_soft_host_rows": (ci, []),
    "ncm_hip_set_gemm_tiles": (None, [ci]),
    "ncm_vq_count_rescores": (None, [ci]),
    "ncm_vq_rescore_counts": (None, [ctypes.POINTER(ctypes.c_longlong), ctypes.POINTER(ctypes.c_longlong)]),
    "tensor_alloc": (vp, [ci, ctypes.POINTER(i64)]),
    "tensor_free": (None, [vp]),
    "tensor_numel": (i64, [ci, ctypes.POINTER(i64)]),
    "tensor_to_host": (None, [vp, vp]),
    "tensor_to_backend": (None, [vp, vp]),
    "mem_d2h": (None, [vp, vp, sz]),
    "mem_h2d": (None, [vp, vp, sz]),
    "mem_d2d": (None, [vp, vp, sz]),
    "arena_init": (None, [sz]),
    "arena_init_default": (None, []),
    "arena_alloc": (vp, [sz]),
    "arena_reset": (None, []),
    "arena_free": (None, []),
    "parena_init": (None, [sz]),
    "parena_alloc": (vp, [sz]),
    "backend_to_host": (vp, [vp, sz]),
    "linear_fwd": (None, [vp, vp, vp, vp, i64, ci, ci]),
    "linear_fwd_ep": (None, [vp, vp, vp, vp, vp, i64, ci, ci, ci]),
    "linear_fwd_glu": (None, [vp, vp, vp, vp, vp, i64, ci, ci, ci]),
    "linear_fwd_gated": (None, [vp, vp, vp, vp, vp, vp, i64, ci, ci, ci]),
    "linear_bwd": (None, [vp, vp, vp, vp, vp, vp, i64, ci, ci]),
    "ncm_hip_linear_plan": (ci, [ci, i64, ci, ci, ctypes.c_char_p, sz]),
    "rowwise_l2sq": (None, [vp, vp, vp, i64, i64, ci]),
    "vq_argmin": (None, [vp, vp, vp, i64, ci, ci]),
    "vq_argmin_noalloc": (ci, [vp, vp, vp, i64, ci, ci]),
    "vq_quantize_multiscale": (None, [vp, ctypes.POINTER(vp), ctypes.POINTER(ci), ci, ci, ci, ci,
                                      vp, vp, vp]),
    "rmsnorm_fwd": (None, [vp, vp, vp, i64, ci]),
    "layernorm_fwd": (None, [vp, vp, vp, vp, i64, ci]),
    "layernorm_eps_fwd": (None, [vp, vp, vp, vp, i64, ci, ctypes.c_float]),
    "gelu_fwd": (None, [vp, vp, i64]),
    "gelu_tanh_fwd": (None, [vp, vp, i64]),
    "silu_fwd": (None, [vp, vp, i64]),
    "rope_apply": (None, [vp, vp, vp, vp, ci, ci, ci, ci]),
    "rope_apply_gqa": (None, [vp, vp, vp, vp, ci, ci, ci, ci, ci]),
    "heads_transpose_fwd": (None, [vp, vp, i64, ci, ci]),
    "heads_transpose_fwd_b": (None, [vp, vp, ci, i64, ci, ci]),
    "sdpa_fwd": (None, [vp, vp, vp, vp, vp, ci, ci, ci, ci, ci]),
    "sdpa_fwd_gqa": (None, [vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci]),
    "sdpa_fwd_gqa_merged": (None, [vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci]),
    "sdpa_fwd_gqa_causal": (None, [vp, vp, vp, vp, ci, ci, ci, ci, ci, ci]),
    "embedding_fwd": (None, [vp, vp, vp, i64, ci]),
    "embedding_fwd_v": (None, [vp, ci, vp, vp, i64, ci]),
    "add_fwd": (None, [vp, vp, vp, i64]),
    "scale_fwd": (None, [vp, ctypes.c_float, vp, i64]),
    "mul_fwd": (None, [vp, vp, vp, i64]),
    "add_inplace_fwd": (None, [vp, vp, i64]),
    "qkv_split_fwd": (None, [vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci]),
    "qkv_split_rope_fwd": (None, [vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci]),
    "head_merge_fwd": (None, [vp, vp, ci, ci, ci, ci, ci]),
    "layernorm_bwd": (None, [vp, vp, vp, vp, vp, vp, i64, ci, ctypes.c_double]),
    "rmsnorm_bwd": (None, [vp, vp, vp, vp, vp, i64, ci]),
    "ce_fwd": (None, [vp, vp, vp, vp, vp, i64, ci]),
    "ce_bwd": (None, [vp, vp, vp, vp, i64, ci, ctypes.c_double]),
    "ce_fwd_bwd": (None, [vp, vp, vp, vp, vp, i64, ci, ctypes.c_double]),
    "sdpa_probs_gqa": (None, [vp, vp, vp, vp, ci, ci, ci, ci, ci, ci]),
    "sdpa_bwd_gqa": (None, [vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci]),
    "adamw_update": (None, [vp, vp, vp, vp, i64] + [ctypes.c_double] * 7),
    "sched_cosine_warmup": (ctypes.c_double, [ctypes.c_long, ctypes.c_double, ctypes.c_double]),
    "grad_clip_global": (ctypes.c_double, [ctypes.POINTER(vp), ctypes.POINTER(i64), ci, ctypes.c_double]),
    "gelu_bwd": (None, [vp, vp, vp, i64]),
    "silu_bwd": (None, [vp, vp, vp, i64]),
    "gelu_tanh_bwd": (None, [vp, vp, vp, i64]),
    "mul_bwd": (None, [vp, vp, vp, vp, vp, i64]),
    "rope_bwd_gqa": (None, [vp] * 6 + [ci] * 5),
    "embedding_bwd": (None, [vp, vp, i64, ci, vp, ci]),
    "qkv_split_bwd": (None, [vp] * 4 + [ci] * 7),
    "head_merge_bwd": (None, [vp, vp] + [ci] * 5),
    "heads_transpose_bwd": (None, [vp, vp] + [ci] * 5),
    "ncm_tape_new": (vp, []),
    "ncm_tape_free": (None, [vp]),
    "ncm_tape_clear": (None, [vp]),
    "ncm_tape_size": (ci, [vp]),
    "ncm_tape_backward": (None, [vp, vp]),
    "ncm_tape_grad": (vp, [vp, vp]),
    "ncm_t_linear": (None, [vp] * 5 + [i64, ci, ci]),
    "ncm_t_embed": (None, [vp, vp, vp, ci, vp, i64, ci]),
    "ncm_t_layernorm": (None, [vp] * 5 + [i64, ci]),
    "ncm_t_layernorm_eps": (None, [vp] * 5 + [i64, ci, ctypes.c_double]),
    "ncm_t_rmsnorm": (None, [vp] * 4 + [i64, ci]),
    "ncm_t_gelu": (None, [vp, vp, vp, i64]),
    "ncm_t_gelu_tanh": (None, [vp, vp, vp, i64]),
    "ncm_t_silu": (None, [vp, vp, vp, i64]),
    "ncm_t_mul": (None, [vp] * 4 + [i64]),
    "ncm_t_add": (None, [vp] * 4 + [i64]),
    "ncm_t_scale": (None, [vp, vp, ctypes.c_float, vp, i64]),
    "ncm_t_rope": (None, [vp] * 7 + [ci] * 5),
    "ncm_t_sdpa": (None, [vp] * 6 + [ci] * 6),
    "ncm_t_sdpa_causal": (None, [vp] * 5 + [ci] * 6),
    "ncm_t_linear_act": (None, [vp] * 6 + [i64, ci, ci, ci]),
    "ncm_t_linear_res": (None, [vp] * 6 + [i64, ci, ci]),
    "ncm_t_linear_qkvsplit": (None, [vp] * 8 + [ci] * 7),
    "ncm_t_sdpa_causal_merge": (None, [vp] * 6 + [ci] * 5),
    "ncm_t_qkvsplit": (None, [vp] * 5 + [ci] * 7),
    "ncm_t_headmerge": (None, [vp] * 3 + [ci] * 5),
    "ncm_t_headsplit": (None, [vp] * 3 + [ci] * 5),
    "ncm_t_ce": (None, [vp] * 6 + [i64, ci, ctypes.c_double]),
    "ncm_gpt2_param_count": (ci, [vp]),
    "ncm_gpt2_param_shape": (i64, [vp, ci, ctypes.POINTER(i64), ctypes.POINTER(i64)]),
    "ncm_gpt2_forward": (vp, [vp, vp, vp, vp, ci, ci]),
    "ncm_gpt2_train_step": (ctypes.c_float, [vp] * 8 + [ci, ci, ctypes.c_long] + [ctypes.c_double] * 4
                            + [ctypes.POINTER(ctypes.c_double)]),
    "ncm_qwen_param_count": (ci, [vp]),
    "ncm_qwen_param_shape": (i64, [vp, ci, ctypes.POINTER(i64), ctypes.POINTER(i64)]),
    "ncm_qwen_new": (vp, [vp, vp]),
    "ncm_qwen_free": (None, [vp]),
    "ncm_qwen_forward": (vp, [vp, vp, ci, ci]),
    "ncm_qwen_decode": (vp, [vp, ci, ci]),
    "ncm_qwen_generate": (ci, [vp, vp, ci, ci, ci, vp]),
    "ncm_qwen_generate_sample": (ci, [vp, vp, ci, ci, ci, ctypes.c_float, ci, ctypes.c_float,
                                      ctypes.POINTER(ctypes.c_uint64), vp, ctypes.POINTER(ci)]),
    "ncm_ncp_param_count": (ci, [vp]),
    "ncm_ncp_param_shape": (i64, [vp, ci, ctypes.POINTER(i64), ctypes.POINTER(i64)]),
    "ncm_ncp_rope_tables": (ci, [ci, ci, ci, vp, vp]),
    "ncm_ncp_forward": (vp, [vp, vp, vp, ci, ci]),
    "argmax_row": (ci, [vp, ci]),
    "argmax_rows": (None, [vp, vp, i64, ci]),
    "rng_next": (ctypes.c_uint64, [ctypes.POINTER(ctypes.c_uint64)]),
    "sample_topkp": (ci, [vp, ci, ctypes.c_float, ci, ctypes.c_float, ctypes.POINTER(ctypes.c_uint64)]),
    "ncm_hip_sample_flag": (ci, []),
    "sample_topkp_dev": (None, [vp, ci, ctypes.c_float, ci, ctypes.c_float, vp, vp, vp]),
    "vq_load": (vp, [vp, vp, ctypes.c_char_p]),
    "ncp_load": (vp, [vp, vp, vp]),
    "ncp_free": (None, [vp]),
    "ncp_forward": (None, [vp, vp, vp, vp, ci]),
    "ncp_P": (ci, [vp]),
    "ncp_T": (ci, [vp]),
    "ncp_ntgt": (ci, [vp]),
    "ncp_lvlfirst": (ci, [vp]),
    "ncp_rope_cos": (vp, [vp]),
    "ncp_rope_sin": (vp, [vp]),
    "ncp_rope_gen_cos": (vp, [vp, ci]),
    "ncp_rope_gen_sin": (vp, [vp, ci]),
    "vq_free": (None, [vp]),
    "vq_total_codes": (ci, [vp]),
    "vq_nlevels": (ci, [vp]),
    "vq_level_len": (ci, [vp, ci]),
    "vq_level_V": (ci, [vp, ci]),
    "vq_Ltotal": (ci, [vp]),
    "vq_Ddim": (ci, [vp]),
    "vq_z_to_idx": (None, [vp, vp, ci, vp]),
    "vq_z_to_idx_soft": (None, [vp, vp, ci, vp, ci, ctypes.c_double, vp]),
    "vq_ema_init": (None, [vp]),
    "vq_ema_update": (None, [vp, vp, vp, ci, ctypes.c_double, ctypes.c_double]),
    "vq_z_to_idx_dev": (None, [vp, vp, ci, vp, vp, vp]),
    "vq_idx_to_zhats": (None, [vp, vp, ci, ctypes.POINTER(vp)]),
    "vq_next_input": (None, [vp, vp, ci, vp, vp, ci]),
    "vq_idx_to_ncm_input": (None, [vp, vp, ci, vp]),
}

# On-disk formats, the AdamW object and NCK1 checkpoints: the reference's
# prototypes (ncm.h:57-70, 139, 262-265, 416-466, 537-540), so the same table
# binds the reference library in the parity tests.
c_dbl = ctypes.c_double
cp = ctypes.c_char_p
FORMAT_SIGS = {
    "weights_load": (ci, [vp, cp]),
    "weights_free": (None, [vp]),
    "weights_get": (vp, [vp, cp]),
    "weights_save": (ci, [vp, cp]),
    "config_load": (ci, [vp, cp]),
    "train_data_load": (vp, [cp, ci]),
    "train_data_free": (None, [vp]),
    "adamw_new": (vp, [vp, vp]),
    "adamw_zero_grad": (None, [vp]),
    "adamw_step": (None, [vp, c_dbl, c_dbl, c_dbl]),
    "adamw_free": (None, [vp]),
    "adamw_sync_to_host": (None, [vp]),
    "ckpt_probe": (ci, [cp]),
    "ckpt_file_hash": (ctypes.c_uint64, [cp, ctypes.POINTER(ctypes.c_uint64)]),
    "ckpt_save_atomic": (ci, [vp, vp, vp, cp, cp, sz]),
    "ckpt_load_training": (ci, [cp, vp, vp, vp, vp, cp, sz]),
    "ckpt_info": (ci, [cp]),
    "ckpt_load_weights_only": (ci, [cp, vp, cp, sz]),
}
_SIGS.update(FORMAT_SIGS)


class NcmError(RuntimeError):
    pass


def header_functions(path=HEADER):
    """Names of the functions include/ncm_hip.h declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b([a-z_][A-Za-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("defined",)))


_lib = None


def load(path=LIB_PATH):
    """Loads libncmhip.so (raises if it was not built) and binds every symbol."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    lib.ncm_hip_set_error_mode(1)  # NCM_ERR_RECORD: raise here instead of exit(1)
    _lib = lib
    return lib


def check():
    lib = load()
    buf = ctypes.create_string_buffer(512)
    code = lib.ncm_hip_last_error(buf, 512)
    if code:
        raise NcmError(f"ncmhip error {code}: {buf.value.decode()}")


def init(device=0):
    lib = load()
    lib.ncm_hip_init(device)
    check()


def sync():
    load().ncm_hip_sync()
    check()


def stream():
    s = load().ncm_hip_stream()
    check()
    return s


class DeviceBuffer:
    """A device allocation made by libncmhip (ncm_hip_malloc)."""

    def __init__(self, nbytes, dtype=np.float32, shape=None):
        lib = load()
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = shape if shape is not None else (self.nbytes // self.dtype.itemsize,)
        self.ptr = lib.ncm_hip_malloc(max(self.nbytes, 16))
        check()

    @classmethod
    def from_numpy(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes, arr.dtype, arr.shape)
        if arr.nbytes:
            load().mem_h2d(b.ptr, arr.ctypes.data, arr.nbytes)
            check()
        return b

    @classmethod
    def empty(cls, shape, dtype=np.float32):
        shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        n = int(np.prod(shape)) if shape else 1
        return cls(n * np.dtype(dtype).itemsize, dtype, shape)

    def upload(self, arr):
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        assert arr.nbytes <= self.nbytes
        load().mem_h2d(self.ptr, arr.ctypes.data, arr.nbytes)
        check()

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        if out.nbytes:
            load().mem_d2h(out.ctypes.data, self.ptr, out.nbytes)
            check()
        return out

    def free(self):
        if self.ptr:
            load().ncm_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _p(b):
    return None if b is None else (b.ptr if isinstance(b, DeviceBuffer) else b)


def linear_fwd(x, W, b, y, batch, M, K, res=None, act="none"):
    lib = load()
    if res is None and act == "none":
        lib.linear_fwd(_p(x), _p(W), _p(b), _p(y), batch, M, K)
    else:
        lib.linear_fwd_ep(_p(x), _p(W), _p(b), _p(res), _p(y), batch, M, K, ACT[act])
    check()


def linear_bwd(x, W, dy, dx, dW, db, batch, M, K):
    load().linear_bwd(_p(x), _p(W), _p(dy), _p(dx), _p(dW), _p(db), batch, M, K)
    check()


def linear_plan(op, batch, M, K):
    """(kernel name, split count) a linear call launches; op in fwd/dx/dw, or
    dwdb for dW and db requested by one linear_bwd call."""
    buf = ctypes.create_string_buffer(64)
    s = load().ncm_hip_linear_plan({"fwd": 0, "dx": 1, "dw": 2, "dwdb": 3}[op], batch, M, K, buf, 64)
    check()
    return buf.value.decode(), s


def rowwise_l2sq(a, b, d2, rows, cols, C):
    load().rowwise_l2sq(_p(a), _p(b), _p(d2), rows, cols, C)
    check()


def vq_argmin(a, E, idx, rows, V, D):
    load().vq_argmin(_p(a), _p(E), _p(idx), rows, V, D)
    check()


def vq_argmin_noalloc(a, E, idx, rows, V, D):
    """vq_argmin with the library's fixed device scratch (no allocation); returns its status."""
    rc = load().vq_argmin_noalloc(_p(a), _p(E), _p(idx), rows, V, D)
    check()
    return rc


def vq_quantize_multiscale(z, Es, vocabs, B, L, D, idx, z_hat, z_rest):
    n = len(Es)
    eptrs = (vp * n)(*[_p(e) for e in Es])
    vocs = (ci * n)(*vocabs)
    load().vq_quantize_multiscale(_p(z), eptrs, vocs, n, B, L, D, _p(idx), _p(z_hat), _p(z_rest))
    check()


def call(name, *args):
    """Calls any header function; DeviceBuffers are passed as device pointers."""
    r = getattr(load(), name)(*[_p(a) if (a is None or isinstance(a, DeviceBuffer)) else a for a in args])
    check()
    return r


def argmax_rows(x, idx, rows, n):
    load().argmax_rows(_p(x), _p(idx), rows, n)
    check()


def sample_topkp(logits, temp, top_k, top_p, rng):
    """sample_topkp on a HOST row (numpy float32); returns (id, new rng, flag)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    st = ctypes.c_uint64(rng)
    i = load().sample_topkp(x.ctypes.data, x.size, temp, top_k, top_p, ctypes.byref(st))
    check()
    return i, st.value, load().ncm_hip_sample_flag()


def sample_topkp_dev(logits, V, temp, top_k, top_p, rng, out, flag=None):
    """Device sampler: logits, rng (uint64 [1]), out (int32 [1]), flag (int32 [1] or None)."""
    load().sample_topkp_dev(_p(logits), V, temp, top_k, top_p, _p(rng), _p(out), _p(flag))
    check()


# ---- HIP events on the library stream (timing) ----
_hip = None


def _hiprt():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        _hip.hipEventRecord.argtypes = [vp, vp]
        _hip.hipEventSynchronize.argtypes = [vp]
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        _hip.hipEventDestroy.argtypes = [vp]
    return _hip


class Event:
    def __init__(self):
        self.ev = vp()
        rc = _hiprt().hipEventCreate(ctypes.byref(self.ev))
        if rc:
            raise NcmError(f"hipEventCreate: {rc}")

    def record(self):
        rc = _hiprt().hipEventRecord(self.ev, stream())
        if rc:
            raise NcmError(f"hipEventRecord: {rc}")

    def synchronize(self):
        rc = _hiprt().hipEventSynchronize(self.ev)
        if rc:
            raise NcmError(f"hipEventSynchronize: {rc}")

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        rc = _hiprt().hipEventElapsedTime(ctypes.byref(ms), self.ev, end.ev)
        if rc:
            raise NcmError(f"hipEventElapsedTime: {rc}")
        return ms.value


class TensorS(ctypes.Structure):
    """Tensor of include/ncm_hip.h (the reference layout, ncm.h:29-34)."""
    _fields_ = [("data", vp), ("shape", i64 * 4), ("ndim", ci), ("n", i64)]


class NamedTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("t", ctypes.POINTER(TensorS))]


class WeightStore(ctypes.Structure):
    _fields_ = [("items", ctypes.POINTER(NamedTensor)), ("count", ci)]

    def names(self):
        return [self.items[i].name.decode() for i in range(self.count)]


class TrainData(ctypes.Structure):
    _fields_ = [("rows", ctypes.POINTER(ci)), ("n_rows", ci), ("row_len", ci)]


class AdamW(ctypes.Structure):
    """AdamW of include/ncm_hip.h (params/m/v/g are device pointers here)."""
    _fields_ = [("params", ctypes.POINTER(vp)), ("m", ctypes.POINTER(vp)), ("v", ctypes.POINTER(vp)),
                ("g", ctypes.POINTER(vp)), ("sizes", ctypes.POINTER(i64)), ("lr", ctypes.POINTER(c_dbl)),
                ("n", ci), ("b1", c_dbl), ("b2", c_dbl), ("eps", c_dbl), ("wd", c_dbl), ("step", ctypes.c_long)]


class CkptRunState(ctypes.Structure):
    _fields_ = [("global_step", ctypes.c_long), ("batch_rng", ctypes.c_ulonglong), ("base_lr", c_dbl),
                ("warmup", c_dbl), ("total", c_dbl), ("batch_B", ci), ("accum_pending", ci),
                ("n_rows", ctypes.c_long), ("row_len", ci), ("data_hash", ctypes.c_uint64), ("data_path", cp),
                ("conf_hash", ctypes.c_uint64), ("tokenizer_id", cp), ("noise_sd", c_dbl),
                ("train_cfg_json", cp)]


class CkptExpect(ctypes.Structure):
    _fields_ = [("batch_B", ci), ("n_rows", ctypes.c_long), ("row_len", ci), ("data_hash", ctypes.c_uint64),
                ("conf_hash", ctypes.c_uint64), ("tokenizer_id", cp), ("base_lr", c_dbl), ("warmup", c_dbl),
                ("total", c_dbl), ("b1", c_dbl), ("b2", c_dbl), ("eps", c_dbl), ("wd", c_dbl)]


class NCMConfig(ctypes.Structure):
    """NCMConfig of include/ncm_hip.h (the reference layout, ncm.h:75-137)."""
    _fields_ = ([("task", ctypes.c_char * 64)]
                + [(f, ci) for f in ("n_layer", "n_head", "n_embd", "context_length", "prefix_len", "bias",
                                     "raw_token_prefix", "contextual_prefix", "prefix_pad_token_id")]
                + [("vocab_size", ci * 64), ("n_levels_out", ci)]
                + [(f, ci) for f in ("predict_level0", "query_level0", "l0_autoregressive",
                                     "attn_pattern_block_diag", "use_positional_encoding", "use_level_encoding",
                                     "use_rope", "rope_base", "use_qk_norm", "use_flex_attention")]
                + [("rope_theta", c_dbl)]
                + [(f, ci) for f in ("n_kv_heads", "ctx_enabled", "ctx_n_layer", "ctx_vocab", "puc_enabled",
                                     "puc_kernel", "shared_output_head", "shared_head_per_level_bias",
                                     "untied_head_bias", "tie_heads_to_codebook", "tie_heads_learn_scale",
                                     "tie_heads_trainable", "tie_heads_bias", "use_swiglu", "use_geglu", "use_relu2",
                                     "parallel_block", "normformer", "use_layerscale", "use_rezero")]
                + [("layerscale_init", ctypes.c_float), ("dropout", ctypes.c_float)]
                + [(f, ci) for f in ("vq_embed_dim", "vq_in_vocab", "vq_context_length", "vq_n_layers",
                                     "vq_compression", "vq_soft_levels")]
                + [("vq_soft_tau", c_dbl), ("levels", ci * 64), ("n_qlevels", ci), ("vq_vocab", ci * 64),
                   ("quant_resi_ratio", ctypes.c_float)]
                + [(f, ci) for f in ("quant_resi_enabled", "quant_resi_share_mode", "learned_l1_sampling",
                                     "learned_l1_cascade", "learned_l1_cascade_base", "learned_l1_norm",
                                     "learned_l1_norm_final", "learned_all_sampling", "pre_quant_groupnorm",
                                     "vq_qk_norm", "enc_layers", "enc_attn_window", "enc_conv_layers",
                                     "enc_conv_kernel", "enc_positional", "dec_layers", "dec_positional")]
                + [("pre_tok", ctypes.c_char * 16), ("sudoku_size", ci), ("hf_model_id", ctypes.c_char * 128),
                   ("eos_token_id", ci), ("pad_token_id", ci), ("gen_temperature", ctypes.c_float),
                   ("gen_top_k", ci), ("gen_top_p", ctypes.c_float), ("gen_cfg_scale", ctypes.c_float),
                   ("gen_freq", ctypes.c_float), ("gen_mu", ctypes.c_float), ("gen_adj_a", ctypes.c_float),
                   ("gen_adj_w", ci), ("gen_adj_d", ctypes.c_float)])


def bind(lib, sigs):
    """Sets restype/argtypes of `sigs` on a ctypes library; returns it."""
    for name, (res, args) in sigs.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


class Gpt2Config(ctypes.Structure):
    """NcmGpt2Config of include/ncm_hip.h."""
    _fields_ = [("n_layer", ctypes.c_int), ("n_embd", ctypes.c_int), ("n_head", ctypes.c_int),
                ("vocab", ctypes.c_int), ("n_pos", ctypes.c_int)]


def ptr_array(bufs):
    """A C array of device pointers (float *const *) for a list of DeviceBuffers."""
    return (ctypes.c_void_p * len(bufs))(*[_p(b) for b in bufs])


class QwenConfig(ctypes.Structure):
    """NcmQwenConfig of include/ncm_hip.h."""
    _fields_ = [("n_layer", ctypes.c_int), ("n_embd", ctypes.c_int), ("n_head", ctypes.c_int),
                ("n_kv", ctypes.c_int), ("n_inner", ctypes.c_int), ("vocab", ctypes.c_int),
                ("n_ctx", ctypes.c_int), ("rope_theta", ctypes.c_double)]


class NcpConfig(ctypes.Structure):
    """NcmNcpConfig of include/ncm_hip.h."""
    _fields_ = [("n_layer", ctypes.c_int), ("n_embd", ctypes.c_int), ("n_head", ctypes.c_int),
                ("n_kv", ctypes.c_int), ("n_inner", ctypes.c_int), ("vocab", ctypes.c_int),
                ("rope_base", ctypes.c_int)]


def weight_store(named):
    """A WeightStore of device tensors for {name: array}; returns (store,
    keep-alive list)."""
    items = (NamedTensor * len(named))()
    keep = [items]
    for j, (k, arr) in enumerate(named.items()):
        buf = DeviceBuffer.from_numpy(np.ascontiguousarray(arr, np.float32))
        t = TensorS()
        t.data = buf.ptr
        for a, d in enumerate(arr.shape):
            t.shape[a] = d
        t.ndim, t.n = arr.ndim, int(arr.size)
        items[j].name = k.encode()
        items[j].t = ctypes.pointer(t)
        keep += [buf, t]
    return WeightStore(items, len(named)), keep


def ncm_config(**fields):
    """An NCMConfig with the given fields set (lists fill the array fields)."""
    c = NCMConfig()
    for k, v in fields.items():
        if isinstance(v, (list, tuple)):
            arr = getattr(c, k)
            for i, x in enumerate(v):
                arr[i] = x
        else:
            setattr(c, k, v)
    return c
