"""Python binding of the C ABI (libdataflow.so) through ctypes.

Mirrors the reference's C interface for the native op path: the
Dataflow_Handle vtable (src/dataflow_handle/include/dataflow_handle.h:28-122),
the op skeleton/fingerprint registry (src/set_ops/include/set_native_op_skeletons.h)
and the submit_* op API (src/dataflow_ops/include/dataflow_ops.h:146-215).
Functions keep the C names, argument order and meaning, and return the C
status (0 / -1). Device pointers are plain integers.

Loading fails loudly when the native library is missing: there is no Python
or CPU fallback for any op.
"""
import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG, "lib")
CORE_LIB = os.path.join(LIB_DIR, "libdataflow.so")
CONFIG_LIB = os.path.join(LIB_DIR, "libdataflow_hip_config.so")
KERNELS = os.path.join(LIB_DIR, "dataflow_kernels_gfx950.hsaco")
MATMUL_LIB = os.path.join(LIB_DIR, "libdataflow_hipblaslt.so")
NOALLOC_LIB = os.path.join(LIB_DIR, "libdataflow_noalloc.so")
# measurement only: streaming copies bench.py times as the memory ceiling
BENCH_COPY_KERNELS = os.path.join(LIB_DIR, "bench_stream_copy_gfx950.hsaco")

# ---- enums (values are part of op fingerprints; never reorder) ----
DATAFLOW_NONE, DATAFLOW_VOID, DATAFLOW_FP64, DATAFLOW_FP32, DATAFLOW_FP16, DATAFLOW_BF16 = range(6)
DATAFLOW_FP8E4M3, DATAFLOW_FP8E5M2, DATAFLOW_UINT64, DATAFLOW_UINT32, DATAFLOW_UINT16, DATAFLOW_UINT8 = range(6, 12)
DATAFLOW_LONG, DATAFLOW_INT, DATAFLOW_BOOL = range(12, 15)
(DATAFLOW_FP64_SCALAR, DATAFLOW_FP32_SCALAR, DATAFLOW_FP16_SCALAR, DATAFLOW_BF16_SCALAR, DATAFLOW_FP8E4M3_SCALAR,
 DATAFLOW_FP8E5M2_SCALAR, DATAFLOW_UINT64_SCALAR, DATAFLOW_UINT32_SCALAR, DATAFLOW_UINT16_SCALAR, DATAFLOW_UINT8_SCALAR,
 DATAFLOW_LONG_SCALAR, DATAFLOW_INT_SCALAR, DATAFLOW_BOOL_SCALAR) = range(15, 28)

COMPUTE_NONE, COMPUTE_CPU, COMPUTE_CUDA, COMPUTE_HSA, COMPUTE_LEVEL_ZERO = range(5)

MAX_OP_ARGS = 32
MAX_OP_NICKNAME_SIZE = 255
MAX_STREAMS = 256
MAX_NATIVE_FUNCTION_LIBS = 1024

NUMPY_DTYPES = {DATAFLOW_FP32: np.float32, DATAFLOW_FP16: np.float16, DATAFLOW_BF16: np.uint16}


# ---- structs (layouts of include/*.h) ----
class OpSkeletonHeader(ctypes.Structure):
    _fields_ = [("op_nickname", ctypes.c_char * (MAX_OP_NICKNAME_SIZE + 1)),
                ("num_args", ctypes.c_int),
                ("arg_dtypes", ctypes.c_int * MAX_OP_ARGS)]


class OpSkeleton(ctypes.Structure):
    _fields_ = [("header", OpSkeletonHeader), ("fingerprint", ctypes.c_uint8 * 32)]


class Op(ctypes.Structure):
    _fields_ = [("op_skeleton", OpSkeleton), ("op_args", ctypes.c_void_p * MAX_OP_ARGS)]


HashFunc = ctypes.CFUNCTYPE(ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64)


class TableConfig(ctypes.Structure):
    _fields_ = [("min_size", ctypes.c_uint64), ("max_size", ctypes.c_uint64),
                ("load_factor", ctypes.c_float), ("shrink_factor", ctypes.c_float),
                ("hash_func", ctypes.c_void_p), ("key_size_bytes", ctypes.c_uint64),
                ("value_size_bytes", ctypes.c_uint64)]


class Table(ctypes.Structure):
    _fields_ = [("cnt", ctypes.c_uint64), ("size", ctypes.c_uint64), ("config", TableConfig),
                ("is_empty_bit_vector", ctypes.c_void_p), ("items", ctypes.c_void_p)]


_VTABLE = ["register_native_code", "register_external_code", "submit_op", "submit_host_op",
           "get_stream_state", "submit_dependency", "sync_stream", "sync_handle",
           "alloc_mem", "free_mem", "set_mem", "enable_access_to_host_mem", "disable_access_to_host_mem",
           "enable_access_to_peer_mem", "disable_access_to_peer_mem",
           "submit_inbound_transfer", "submit_outbound_transfer", "submit_peer_transfer"]


class DataflowHandle(ctypes.Structure):
    _fields_ = [("compute_type", ctypes.c_int), ("device_id", ctypes.c_int),
                ("device_handle", ctypes.c_void_p), ("device_info", ctypes.c_void_p),
                ("ctx_id", ctypes.c_int), ("ctx", ctypes.c_void_p),
                ("num_streams", ctypes.c_int), ("streams", ctypes.c_void_p),
                ("stream_prios", ctypes.c_int * MAX_STREAMS), ("stream_names", ctypes.c_char_p * MAX_STREAMS),
                ("stream_states", ctypes.c_void_p),
                ("num_native_function_libs", ctypes.c_int),
                ("native_function_libs", ctypes.c_void_p * MAX_NATIVE_FUNCTION_LIBS),
                ("num_ops", ctypes.c_int), ("op_table", Table)] + [(n, ctypes.c_void_p) for n in _VTABLE]


class HipDeviceInfo(ctypes.Structure):
    _fields_ = [("total_mem", ctypes.c_size_t), ("arch_num", ctypes.c_int), ("cu_count", ctypes.c_int),
                ("max_threads_per_block", ctypes.c_int), ("max_smem_per_block", ctypes.c_int),
                ("optin_max_smem_per_block", ctypes.c_int), ("host_numa_id", ctypes.c_int),
                ("warp_size", ctypes.c_int), ("num_xcds", ctypes.c_int), ("l2_bytes", ctypes.c_int),
                ("arch_name", ctypes.c_char * 64)]


_P = ctypes.c_void_p
_H = ctypes.POINTER(DataflowHandle)
_VT_TYPES = {
    "submit_op": ctypes.CFUNCTYPE(ctypes.c_int, _H, ctypes.POINTER(Op), ctypes.c_int),
    "sync_stream": ctypes.CFUNCTYPE(ctypes.c_int, _H, ctypes.c_int),
    "sync_handle": ctypes.CFUNCTYPE(ctypes.c_int, _H),
    "alloc_mem": ctypes.CFUNCTYPE(_P, _H, ctypes.c_uint64),
    "free_mem": ctypes.CFUNCTYPE(None, _H, _P),
    "set_mem": ctypes.CFUNCTYPE(ctypes.c_int, _H, ctypes.c_int, _P, ctypes.c_uint8, ctypes.c_uint64),
    "submit_inbound_transfer": ctypes.CFUNCTYPE(ctypes.c_int, _H, ctypes.c_int, _P, _P, ctypes.c_uint64),
    "submit_outbound_transfer": ctypes.CFUNCTYPE(ctypes.c_int, _H, ctypes.c_int, _P, _P, ctypes.c_uint64),
    "submit_peer_transfer": ctypes.CFUNCTYPE(ctypes.c_int, _H, ctypes.c_int, _P, _P, ctypes.c_uint64),
    "get_stream_state": ctypes.CFUNCTYPE(_P, _H, ctypes.c_int),
    "submit_dependency": ctypes.CFUNCTYPE(ctypes.c_int, _H, ctypes.c_int, _P),
    "submit_host_op": ctypes.CFUNCTYPE(ctypes.c_int, _H, _P, _P, ctypes.c_int),
}

# host functions for submit_host_op: void fn(void * arg)
HostFunc = ctypes.CFUNCTYPE(None, ctypes.c_void_p)

# ---- library ----
_lib = None


def lib():
    """The loaded libdataflow.so (raises when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(CORE_LIB):
            raise RuntimeError("native library %s is missing: run __graft_entry__.build() first" % CORE_LIB)
        _lib = ctypes.CDLL(CORE_LIB)
        _declare(_lib)
    return _lib


def _declare(L):
    i, u64, f32, vp = ctypes.c_int, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p
    L.dataflow_sizeof_element.restype = ctypes.c_size_t
    L.dataflow_sizeof_element.argtypes = [i]
    L.dataflow_datatype_as_string.restype = ctypes.c_char_p
    L.dataflow_datatype_as_string.argtypes = [i]
    L.dataflow_convert_datatype.argtypes = [vp, vp, i, i, ctypes.c_long, i]
    L.do_fingerprinting.argtypes = [vp, u64, vp, i]
    L.do_fingerprinting.restype = None
    L.fingerprint_to_least_sig64.restype = u64
    L.fingerprint_to_least_sig64.argtypes = [vp, i]
    L.get_fingerprint_num_bytes.restype = ctypes.c_uint8
    L.set_native_op_skeleton.argtypes = [ctypes.POINTER(OpSkeleton), ctypes.c_char_p, i, i]
    L.init_dataflow_handle.argtypes = [_H, i, i, i, ctypes.c_uint, i, vp, vp]
    L.init_hip_dataflow_handle.argtypes = [_H, i, i, i, ctypes.c_uint, i, vp, vp]
    L.destroy_dataflow_handle.argtypes = [_H]
    L.register_native_ops.argtypes = [_H, ctypes.c_char_p, ctypes.c_char_p]
    h, s = _H, i
    L.register_external_matmul.argtypes = [_H, ctypes.c_char_p]
    L.submit_matmul.argtypes = [h, s, i, i, i, i, i, i, i, i, i, i, f32, f32, vp, vp, vp, vp, u64, vp]
    L.submit_transformer_head.argtypes = [h, s, s] + [vp] * 8
    L.submit_embedding.argtypes = [h, s, i, i, i, vp, vp, vp]
    L.submit_copy_to_seq_context.argtypes = [h, s, i, u64, i, i, vp, vp, vp, vp, vp]
    L.submit_rms_norm.argtypes = [h, s, i, i, i, f32, vp, vp, vp, vp, vp]
    L.submit_rms_norm_bwd_x.argtypes = [h, s, i, i, i, i, f32, vp, vp, vp, vp, vp, vp]
    L.submit_rms_norm_bwd_w.argtypes = [h, s, i, i, i, i, f32, vp, vp, vp, vp]
    L.submit_rms_norm_bwd.argtypes = [h, s, i, i, i, i, f32, vp, vp, vp, vp, vp, vp]
    L.submit_rope.argtypes = [h, s, i, u64, i, i, i, i, vp, vp, vp]
    L.submit_rope_copy_to_seq_context.argtypes = [h, s, i, u64, i, i, i, i, vp, vp, vp, vp, vp, vp]
    L.submit_rope_bwd_x.argtypes = [h, s, i, u64, i, i, i, i, vp, vp, vp]
    L.submit_swiglu.argtypes = [h, s, i, i, i, vp, vp, vp]
    L.submit_swiglu_bwd_x.argtypes = [h, s, i, i, i, i, vp, vp, vp, vp, vp]
    L.submit_softmax.argtypes = [h, s, i, i, i, i, vp, vp]
    L.submit_cross_entropy_loss.argtypes = [h, s, i, i, i, vp, vp]
    L.submit_softmax_cross_entropy_loss.argtypes = [h, s, i, i, i, vp, vp, vp, vp]


_noalloc = None


def noalloc_lib():
    """The loaded libdataflow_noalloc.so (raises when it has not been built)."""
    global _noalloc
    if _noalloc is None:
        if not os.path.exists(NOALLOC_LIB):
            raise RuntimeError("native library %s is missing: run __graft_entry__.build() first" % NOALLOC_LIB)
        lib()   # its dependency, loaded from the same directory
        L = ctypes.CDLL(NOALLOC_LIB)
        i, f32, vp = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
        L.dataflow_rms_norm_bwd_noalloc.argtypes = [vp, i, i, i, i, f32, vp, vp, vp, vp, vp, vp]
        L.dataflow_rms_norm_bwd_noalloc.restype = i
        _noalloc = L
    return _noalloc


def rms_norm_bwd_noalloc(stream, fwd_dt, bwd_dt, n_rows, n_cols, eps, fwd_rms_vals, rms_weight, X_inp, upstream_dX, dX, dW):
    """dataflow_rms_norm_bwd_noalloc (include/dataflow_noalloc.h): submit_rms_norm_bwd's
    computation on a hipStream_t, with no handle and no allocation."""
    return noalloc_lib().dataflow_rms_norm_bwd_noalloc(stream, fwd_dt, bwd_dt, n_rows, n_cols, eps, fwd_rms_vals,
                                                       rms_weight, X_inp, upstream_dX, dX, dW)


def datatype_as_string(dt):
    return lib().dataflow_datatype_as_string(dt).decode()


def sizeof_element(dt):
    return lib().dataflow_sizeof_element(dt)


def native_op_skeleton(op_name, fwd_dt, bwd_dt=DATAFLOW_NONE):
    """Op_Skeleton for a native op (set_native_op_skeleton); raises on unknown ops."""
    sk = OpSkeleton()
    if lib().set_native_op_skeleton(ctypes.byref(sk), op_name.encode(), fwd_dt, bwd_dt) != 0:
        raise ValueError("unknown native op %r" % op_name)
    return sk


def header_bytes(sk):
    return bytes(ctypes.string_at(ctypes.addressof(sk.header), ctypes.sizeof(OpSkeletonHeader)))


class Handle:
    """A Dataflow_Handle on one AMD GPU (COMPUTE_HSA) with the native ops registered."""

    def __init__(self, device_id=0, num_streams=1, register=True, matmul=False):
        self.h = DataflowHandle()
        L = lib()
        if L.init_dataflow_handle(ctypes.byref(self.h), COMPUTE_HSA, device_id, 0, 0, num_streams, None, None) != 0:
            raise RuntimeError("init_dataflow_handle failed for device %d" % device_id)
        self._alive = True
        self._fns = {n: ctypes.cast(getattr(self.h, n), t) for n, t in _VT_TYPES.items()}
        self.num_registered = 0
        if register:
            n = L.register_native_ops(ctypes.byref(self.h), KERNELS.encode(), CONFIG_LIB.encode())
            if n <= 0:
                raise RuntimeError("register_native_ops failed (%d)" % n)
            self.num_registered = n
        if matmul:
            if L.register_external_matmul(ctypes.byref(self.h), MATMUL_LIB.encode()) != 1:
                raise RuntimeError("register_external_matmul failed (%s)" % MATMUL_LIB)
            self.num_registered += 1

    @property
    def ref(self):
        return ctypes.byref(self.h)

    @property
    def device_info(self):
        return ctypes.cast(self.h.device_info, ctypes.POINTER(HipDeviceInfo)).contents

    def stream(self, stream_id=0):
        """hipStream_t (as an int) of one of the handle's streams."""
        return ctypes.cast(self.h.streams, ctypes.POINTER(ctypes.c_void_p))[stream_id]

    def submit_op(self, op, stream_id=0):
        return self._fns["submit_op"](self.ref, ctypes.byref(op), stream_id)

    def alloc(self, nbytes):
        p = self._fns["alloc_mem"](self.ref, max(int(nbytes), 1))
        if not p:
            raise MemoryError("alloc_mem(%d) failed" % nbytes)
        return p

    def free(self, ptr):
        self._fns["free_mem"](self.ref, ptr)

    def set_mem(self, ptr, val, nbytes, stream_id=-1):
        return self._fns["set_mem"](self.ref, stream_id, ptr, val, nbytes)

    def to_device(self, arr, ptr=None, stream_id=-1):
        arr = np.ascontiguousarray(arr)
        if ptr is None:
            ptr = self.alloc(arr.nbytes)
        if arr.nbytes and self._fns["submit_inbound_transfer"](self.ref, stream_id, ptr, arr.ctypes.data, arr.nbytes) != 0:
            raise RuntimeError("inbound transfer failed")
        return ptr

    def to_host(self, ptr, shape, dtype, stream_id=-1):
        out = np.empty(shape, dtype=dtype)
        if out.nbytes and self._fns["submit_outbound_transfer"](self.ref, stream_id, out.ctypes.data, ptr, out.nbytes) != 0:
            raise RuntimeError("outbound transfer failed")
        return out

    def copy(self, dst, src, nbytes, stream_id=-1):
        return self._fns["submit_peer_transfer"](self.ref, stream_id, dst, src, nbytes)

    def stream_state(self, stream_id):
        """get_stream_state: an event recorded now on the stream (NULL on error)."""
        return self._fns["get_stream_state"](self.ref, stream_id)

    def submit_dependency(self, stream_id, state):
        """submit_dependency: the stream waits for a state from stream_state."""
        return self._fns["submit_dependency"](self.ref, stream_id, state)

    def submit_host_op(self, fn, arg, stream_id=0):
        """submit_host_op: `fn` (a HostFunc; the caller keeps it alive) runs on a
        runtime thread once the stream's earlier work is done."""
        return self._fns["submit_host_op"](self.ref, ctypes.cast(fn, ctypes.c_void_p), arg, stream_id)

    def sync_stream(self, stream_id=0):
        return self._fns["sync_stream"](self.ref, stream_id)

    def sync(self):
        return self._fns["sync_handle"](self.ref)

    def destroy(self):
        if self._alive:
            lib().destroy_dataflow_handle(self.ref)
            self._alive = False


# ---- op API: same names, argument order and status as the C functions ----
def _h(handle):
    return handle.ref if isinstance(handle, Handle) else handle


def submit_rms_norm(handle, stream_id, fwd_dt, n_rows, n_cols, eps, rms_weight, X, out, weighted_sums, rms_vals):
    return lib().submit_rms_norm(_h(handle), stream_id, fwd_dt, n_rows, n_cols, eps, rms_weight, X, out, weighted_sums, rms_vals)


def submit_rms_norm_bwd_x(handle, stream_id, fwd_dt, bwd_dt, n_rows, n_cols, eps, fwd_weighted_sums, fwd_rms_vals,
                          rms_weight, X_inp, upstream_dX, dX):
    return lib().submit_rms_norm_bwd_x(_h(handle), stream_id, fwd_dt, bwd_dt, n_rows, n_cols, eps, fwd_weighted_sums,
                                       fwd_rms_vals, rms_weight, X_inp, upstream_dX, dX)


def submit_rms_norm_bwd_w(handle, stream_id, fwd_dt, bwd_dt, n_rows, n_cols, eps, fwd_rms_vals, X_inp, upstream_dX, dW):
    return lib().submit_rms_norm_bwd_w(_h(handle), stream_id, fwd_dt, bwd_dt, n_rows, n_cols, eps, fwd_rms_vals,
                                       X_inp, upstream_dX, dW)


def submit_rms_norm_bwd(handle, stream_id, fwd_dt, bwd_dt, n_rows, n_cols, eps, fwd_rms_vals, rms_weight, X_inp,
                        upstream_dX, dX, dW):
    return lib().submit_rms_norm_bwd(_h(handle), stream_id, fwd_dt, bwd_dt, n_rows, n_cols, eps, fwd_rms_vals,
                                     rms_weight, X_inp, upstream_dX, dX, dW)


def submit_matmul(handle, stream_id, a_dt, b_dt, c_dt, d_dt, compute_dt, to_trans_a, to_trans_b, M, K, N, alpha, beta,
                  A, B, C, D, workspaceBytes, workspace):
    return lib().submit_matmul(_h(handle), stream_id, a_dt, b_dt, c_dt, d_dt, compute_dt, to_trans_a, to_trans_b, M, K, N,
                               alpha, beta, A, B, C, D, workspaceBytes, workspace)


class EmbeddingConfig(ctypes.Structure):
    _fields_ = [("vocab_size", ctypes.c_int), ("embedding_size", ctypes.c_int)]


class TransformerHead(ctypes.Structure):
    """transformer_head.h (layout of the reference's Transformer_Head)"""
    _fields_ = [("fwd_dt", ctypes.c_int), ("bwd_dt", ctypes.c_int), ("compute_dt", ctypes.c_int), ("eps", ctypes.c_float),
                ("embedding_config", EmbeddingConfig), ("buffer", ctypes.c_void_p), ("w_head_norm", ctypes.c_void_p),
                ("w_head", ctypes.c_void_p)]


class TransformerHeadActivations(ctypes.Structure):
    _fields_ = [("num_tokens", ctypes.c_int), ("buffer", ctypes.c_void_p), ("head_norm_out", ctypes.c_void_p),
                ("head_norm_weighted_sums", ctypes.c_void_p), ("head_norm_rms_vals", ctypes.c_void_p),
                ("head_out", ctypes.c_void_p), ("kernel_workspace", ctypes.c_void_p),
                ("kernel_workspaceBytes", ctypes.c_uint64)]


class TransformerBlockTransition(ctypes.Structure):
    _fields_ = [("batch_config", ctypes.c_void_p), ("X", ctypes.c_void_p)]


class TransformerModelOutput(ctypes.Structure):
    _fields_ = [("batch_config", ctypes.c_void_p), ("token_ids", ctypes.c_void_p), ("labels", ctypes.c_void_p),
                ("logits", ctypes.c_void_p), ("loss", ctypes.c_void_p), ("loss_avg", ctypes.c_float)]


def submit_transformer_head(handle, compute_stream_id, out_copy_stream_id, block_input, transformer_head, head_activations,
                            model_output, grad_transformer_head=None, grad_head_activations=None, grad_stream=None,
                            next_grad_stream=None):
    ref = lambda x: None if x is None else ctypes.cast(ctypes.byref(x), ctypes.c_void_p)
    return lib().submit_transformer_head(_h(handle), compute_stream_id, out_copy_stream_id, ref(block_input),
                                         ref(transformer_head), ref(head_activations), ref(model_output),
                                         ref(grad_transformer_head), ref(grad_head_activations), ref(grad_stream),
                                         ref(next_grad_stream))


def submit_embedding(handle, stream_id, fwd_dt, num_tokens, embed_dim, token_ids, embedding_table, output):
    return lib().submit_embedding(_h(handle), stream_id, fwd_dt, num_tokens, embed_dim, token_ids, embedding_table, output)


def submit_copy_to_seq_context(handle, stream_id, fwd_dt, N, total_tokens, kv_dim, X_k, X_v, seq_positions,
                               seq_context_ptrs, seq_context_sizes):
    return lib().submit_copy_to_seq_context(_h(handle), stream_id, fwd_dt, N, total_tokens, kv_dim, X_k, X_v,
                                            seq_positions, seq_context_ptrs, seq_context_sizes)


def submit_rope_copy_to_seq_context(handle, stream_id, fwd_dt, N, model_dim, head_dim, num_kv_heads, theta, seq_positions,
                                    X_q, X_k, X_v, seq_context_ptrs, seq_context_sizes):
    """RoPE forward on X_q, X_k in place and the KV-cache scatter of the rotated
    K rows and the X_v rows, in one kernel (no reference counterpart)."""
    return lib().submit_rope_copy_to_seq_context(_h(handle), stream_id, fwd_dt, N, model_dim, head_dim, num_kv_heads, theta,
                                                 seq_positions, X_q, X_k, X_v, seq_context_ptrs, seq_context_sizes)


def submit_rope(handle, stream_id, fwd_dt, N, model_dim, head_dim, num_kv_heads, theta, seq_positions, X_q, X_k):
    return lib().submit_rope(_h(handle), stream_id, fwd_dt, N, model_dim, head_dim, num_kv_heads, theta,
                             seq_positions, X_q, X_k)


def submit_rope_bwd_x(handle, stream_id, bwd_dt, N, model_dim, head_dim, num_kv_heads, theta, seq_positions, dX_q, dX_k):
    return lib().submit_rope_bwd_x(_h(handle), stream_id, bwd_dt, N, model_dim, head_dim, num_kv_heads, theta,
                                   seq_positions, dX_q, dX_k)


def submit_swiglu(handle, stream_id, fwd_dt, num_rows, num_cols, x_w1, x_w3, out):
    return lib().submit_swiglu(_h(handle), stream_id, fwd_dt, num_rows, num_cols, x_w1, x_w3, out)


def submit_swiglu_bwd_x(handle, stream_id, fwd_dt, bwd_dt, num_rows, num_cols, x_w1, x_w3, upstream_dX, dX_w1, dX_w3):
    return lib().submit_swiglu_bwd_x(_h(handle), stream_id, fwd_dt, bwd_dt, num_rows, num_cols, x_w1, x_w3,
                                     upstream_dX, dX_w1, dX_w3)


def submit_softmax(handle, stream_id, fwd_dt, bwd_dt, n_rows, n_cols, X, out):
    return lib().submit_softmax(_h(handle), stream_id, fwd_dt, bwd_dt, n_rows, n_cols, X, out)


def submit_cross_entropy_loss(handle, stream_id, bwd_dt, n_rows, n_cols, pred_logits, labels):
    return lib().submit_cross_entropy_loss(_h(handle), stream_id, bwd_dt, n_rows, n_cols, pred_logits, labels)


def submit_softmax_cross_entropy_loss(handle, stream_id, dt, n_rows, n_cols, logits, labels, loss, mean_loss):
    return lib().submit_softmax_cross_entropy_loss(_h(handle), stream_id, dt, n_rows, n_cols, logits, labels,
                                                   loss, mean_loss)
