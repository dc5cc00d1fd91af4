"""ctypes binding of libnumrs_hip.so (declarations mirror include/numrs_hip.h).

The library is loaded from numrs_amd/lib/ only.  There is no fallback: if it
is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import re

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libnumrs_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG), "include", "numrs_hip.h")

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes)
SIGNATURES = {
    "numrs_hip_create": (_i, [_i, ctypes.POINTER(_vp)]),
    "numrs_hip_destroy": (_i, [_vp]),
    "numrs_hip_last_error": (ctypes.c_char_p, [_vp]),
    "numrs_hip_create_error": (ctypes.c_char_p, []),
    "numrs_hip_device_info": (_i, [_vp, ctypes.POINTER(_i), ctypes.c_char_p, _sz]),
    "numrs_hip_malloc": (_i, [_vp, _sz, ctypes.POINTER(_vp)]),
    "numrs_hip_free": (_i, [_vp, _vp]),
    "numrs_hip_upload": (_i, [_vp, _vp, _vp, _sz]),
    "numrs_hip_download": (_i, [_vp, _vp, _vp, _sz]),
    "numrs_hip_copy": (_i, [_vp, _vp, _vp, _sz]),
    "numrs_hip_fill": (_i, [_vp, _vp, _i64, _f]),
    "numrs_hip_stream_probe": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i, _i]),
    "numrs_hip_sync": (_i, [_vp]),
    "numrs_hip_reserve": (_i, [_vp, _sz]),
    "numrs_hip_stream": (_vp, [_vp]),
    "numrs_hip_timer_record": (_i, [_vp, _i]),
    "numrs_hip_timer_elapsed_ms": (_i, [_vp, _i, _i, ctypes.POINTER(_f)]),
    "numrs_hip_graph_begin": (_i, [_vp]),
    "numrs_hip_graph_end": (_i, [_vp, ctypes.POINTER(_vp)]),
    "numrs_hip_graph_abort": (_i, [_vp]),
    "numrs_hip_graph_launch": (_i, [_vp]),
    "numrs_hip_graph_destroy": (_i, [_vp]),
    "numrs_hip_matmul_backward": (_i, [_vp] * 6 + [_i64] * 3 + [_i]),
    "numrs_hip_matmul_backward_batched": (_i, [_vp] * 6 + [_i64] * 7 + [_i]),
    "numrs_hip_matmul": (_i, [_vp] * 4 + [_i64] * 3 + [_i] * 3),
    "numrs_hip_matmul_batched": (_i, [_vp] * 4 + [_i64] * 7 + [_i] * 3),
    "numrs_hip_linear_forward": (_i, [_vp] * 5 + [_i64] * 3),
    "numrs_hip_linear_backward": (_i, [_vp] * 7 + [_i64] * 3 + [_i] * 4),
    "numrs_hip_linear_relu_forward": (_i, [_vp] * 5 + [_i64] * 3),
    "numrs_hip_linear_relu_backward": (_i, [_vp] * 8 + [_i64] * 3 + [_i] * 4),
    "numrs_hip_linear_residual_forward": (_i, [_vp] * 6 + [_i64] * 3),
    "numrs_hip_linear_gelu_forward": (_i, [_vp] * 6 + [_i64] * 3),
    "numrs_hip_linear_gelu_backward": (_i, [_vp] * 8 + [_i64] * 3 + [_i] * 4),
    "numrs_hip_gemm": (_i, [_vp, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i, _i, _f, _i,
                            _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "numrs_hip_sum_to_shape": (_i, [_vp, _vp, _i64p, _i, _vp, _i64p, _i, _i, _i]),
    "numrs_hip_relu_bias_backward": (_i, [_vp] * 5 + [_i64, _i64, _i, _i]),
    "numrs_hip_relu_bias_backward_noalloc": (_i, [_vp] * 5 + [_i64, _i64, _i, _i]),
    "numrs_hip_unary_backward": (_i, [_vp, _i, _vp, _vp, _vp, _i64, _f, _i]),
    "numrs_hip_binary_backward": (_i, [_vp, _i] + [_vp] * 5 + [_i64, _i]),
    "numrs_hip_fill_grad": (_i, [_vp, _vp, _vp, _i64, _i, _i]),
    "numrs_hip_mse_backward": (_i, [_vp] * 6 + [_i64, _i]),
    "numrs_hip_softmax_ce_backward": (_i, [_vp] * 6 + [_i64, _i64, _i]),
    "numrs_hip_softmax_backward": (_i, [_vp] * 4 + [_i64, _i64, _i]),
    "numrs_hip_reduce_axis": (_i, [_vp, _vp, _i64, _i64, _i64, _i, _vp]),
    "numrs_hip_elementwise": (_i, [_vp, _i, _vp, _vp, _vp, _i64]),
    "numrs_hip_reduction": (_i, [_vp, _i, _vp, _i64p, _i, _i, _vp]),
    "numrs_hip_broadcast_axis": (_i, [_vp, _vp, _i64, _i64, _i64, _i, _vp, _i]),
    "numrs_hip_softmax_axis_forward": (_i, [_vp, _vp, _vp, _i64, _i64, _i64]),
    "numrs_hip_softmax_axis_backward": (_i, [_vp] * 4 + [_i64, _i64, _i64, _i]),
    "numrs_hip_argmax_rows": (_i, [_vp] * 3 + [_i64, _i64, _i]),
    "numrs_hip_sgd_step": (_i, [_vp] * 4 + [_i64, _f, _f, _f]),
    "numrs_hip_adam_step": (_i, [_vp] * 5 + [_i64, _f, _f, _f, _f, _f, _i]),
    "numrs_hip_sgd_step_multi": (_i, [_vp] * 4 + [_i64p, _i, _f, _f, _f]),
    "numrs_hip_adam_step_multi": (_i, [_vp] * 5 + [_i64p, _i, _f, _f, _f, _f, _f, _i]),
    # forward kernels
    "numrs_hip_binary_forward": (_i, [_vp, _i, _vp, _i64p, _i, _vp, _i64p, _i, _vp]),
    "numrs_hip_unary_forward": (_i, [_vp, _i, _vp, _vp, _i64, _f]),
    "numrs_hip_transpose": (_i, [_vp, _vp, _vp, _i64, _i64]),
    "numrs_hip_sum": (_i, [_vp, _vp, _i64, _i, _vp]),
    "numrs_hip_mse_loss": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "numrs_hip_cross_entropy_loss": (_i, [_vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "numrs_hip_softmax_forward": (_i, [_vp, _vp, _vp, _i64, _i64, _f]),
    "numrs_hip_layernorm_forward": (_i, [_vp] * 7 + [_i64, _i64, _f]),
    "numrs_hip_layernorm_backward": (_i, [_vp] * 9 + [_i64, _i64, _i, _i, _i]),
    "numrs_hip_lstm_forward": (_i, [_vp] * 10 + [_i64] * 4),
    "numrs_hip_lstm_backward": (_i, [_vp] * 14 + [_i64] * 4 + [_i] * 4),
    "numrs_hip_lstm2_forward": (_i, [_vp] * 14 + [_i64] * 5),
    "numrs_hip_lstm2_backward": (_i, [_vp] * 20 + [_i64] * 5 + [_i] * 7),
    "numrs_hip_time_slice": (_i, [_vp] * 3 + [_i64] * 4 + [_i, _i]),
    "numrs_hip_attention_forward": (_i, [_vp] * 6 + [_i64] * 4),
    "numrs_hip_attention_backward": (_i, [_vp] * 9 + [_i64] * 4 + [_i]),
    "numrs_hip_attention_forward_strided": (_i, [_vp] * 4 + [_i64, _vp, _vp] + [_i64] * 5),
    "numrs_hip_attention_backward_strided": (_i, [_vp] * 4 + [_i64, _vp, _vp, _i64] + [_vp] * 3 +
                                             [_i64] * 4 + [_i]),
    "numrs_hip_attention_backward_out_strided": (_i, [_vp] * 4 + [_i64, _vp, _vp, _vp, _i64] +
                                                 [_vp] * 3 + [_i64] * 4 + [_i]),
    # tensor engine
    "numrs_hip_set_grad_enabled": (None, [_i]),
    "numrs_hip_is_grad_enabled": (_i, []),
    "numrs_hip_set_unbroadcast_mode": (_i, [_vp, _i]),
    "numrs_hip_set_recurrence_mode": (_i, [_vp, _i]),
    "numrs_hip_set_split_reduction": (_i, [_vp, _i]),
    "numrs_hip_persistent_launches": (_i64, [_vp]),
    "numrs_hip_set_persistent_wait_limit": (_i, [_vp, _i]),
    "numrs_hip_tensor_new": (_i, [_vp, _vp, _i64p, _i, _i, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_free": (_i, [_vp]),
    "numrs_hip_tensor_shape": (_i, [_vp, _i64p, _i]),
    "numrs_hip_tensor_numel": (_i64, [_vp]),
    "numrs_hip_tensor_requires_grad": (_i, [_vp]),
    "numrs_hip_tensor_is_leaf": (_i, [_vp]),
    "numrs_hip_tensor_values": (_i, [_vp, _vp, _i64]),
    "numrs_hip_tensor_gradient": (_i, [_vp, _vp, _i64]),
    "numrs_hip_tensor_set_gradient": (_i, [_vp, _vp, _i64]),
    "numrs_hip_tensor_zero_grad": (_i, [_vp]),
    "numrs_hip_tensor_device_ptrs": (_i, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_backward": (_i, [_vp]),
    "numrs_hip_tensor_detach": (_i, [_vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_binary": (_i, [_i, _vp, _vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_unary": (_i, [_i, _vp, _f, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_matmul": (_i, [_vp, _vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_transpose": (_i, [_vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_reshape": (_i, [_vp, _i64p, _i, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_sum": (_i, [_vp, _i, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_mse_loss": (_i, [_vp, _vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_cross_entropy_loss": (_i, [_vp, _vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_cross_entropy_labels": (_i, [_vp, _vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_softmax": (_i, [_vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_sum_axis": (_i, [_vp, _i64, _i, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_softmax_axis": (_i, [_vp, _i64, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_layer_norm": (_i, [_vp, _vp, _vp, _f, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_linear": (_i, [_vp, _vp, _vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_linear_relu": (_i, [_vp, _vp, _vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_linear_residual": (_i, [_vp, _vp, _vp, _vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_linear_gelu": (_i, [_vp, _vp, _vp, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_lstm": (_i, [_vp] * 4 + [ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_lstm2": (_i, [_vp] * 7 + [ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_time_slice": (_i, [_vp, _i64, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_attention": (_i, [_vp, _vp, _vp, _i64, _i64, _i64, ctypes.POINTER(_vp)]),
    "numrs_hip_tensor_attention_qkv": (_i, [_vp, _i64, _i64, _i64, ctypes.POINTER(_vp)]),
    "numrs_hip_optim_sgd": (_i, [_vp, ctypes.POINTER(_vp), _i, _f, _f, _f, ctypes.POINTER(_vp)]),
    "numrs_hip_optim_adam": (_i, [_vp, ctypes.POINTER(_vp), _i, _f, _f, _f, _f, _f,
                                 ctypes.POINTER(_vp)]),
    "numrs_hip_optim_step": (_i, [_vp]),
    "numrs_hip_optim_zero_grad": (_i, [_vp]),
    "numrs_hip_optim_set_lr": (_i, [_vp, _f]),
    "numrs_hip_optim_lr": (_f, [_vp]),
    "numrs_hip_optim_free": (_i, [_vp]),
    "numrs_hip_optim_state_info": (_i, [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i),
                                        ctypes.POINTER(_i64)]),
    "numrs_hip_optim_state_get": (_i, [_vp, _i, _i, _vp, _i64]),
    "numrs_hip_optim_state_set": (_i, [_vp, _i, _i, _vp, _i64]),
    "numrs_hip_optim_set_step": (_i, [_vp, _i64]),
    "numrs_hip_optimizer_step": (_i, [_vp, _i] + [_vp] * 4 + [_i64p, _i, _vp, _i, _i]),
    "numrs_hip_lookahead_update": (_i, [_vp, _vp, _vp, _i64p, _i, _f]),
    "numrs_hip_dot": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "numrs_hip_optim_create": (_i, [_vp, _i, ctypes.POINTER(_vp), _i, _vp, _i,
                                    ctypes.POINTER(_vp)]),
    "numrs_hip_optim_lookahead": (_i, [_vp, ctypes.POINTER(_vp), _i, _i, _f,
                                       ctypes.POINTER(_vp)]),
    "numrs_hip_optim_lbfgs": (_i, [_vp, ctypes.POINTER(_vp), _i, _f, _i, _i,
                                   ctypes.POINTER(_vp)]),
    "numrs_hip_scheduler_create": (_i, [_i, _vp, _i, ctypes.POINTER(_vp)]),
    "numrs_hip_scheduler_step": (_i, [_vp, _vp]),
    "numrs_hip_scheduler_step_metric": (_i, [_vp, _f, _vp]),
    "numrs_hip_scheduler_get_lr": (_f, [_vp]),
    "numrs_hip_scheduler_free": (_i, [_vp]),
}

# Enum values of include/numrs_hip.h.
OK, E_INVALID, E_SHAPE, E_HIP, E_NOMEM, E_NODEV = 0, -1, -2, -3, -4, -5
UNBROADCAST_CORRECT, UNBROADCAST_REFERENCE = 0, 1
RELU, SIGMOID, TANH, EXP, LOG, GELU, SQRT, SIN, COS, TAN, POW = range(11)
ADD, SUB, MUL, DIV = range(4)
# DispatchTable kinds (llo/elementwise.rs:38-68, llo/reduction.rs:12-19)
(EW_ADD, EW_MUL, EW_SUB, EW_DIV, EW_POW, EW_SQRT, EW_SIN, EW_COS, EW_TAN, EW_ASIN, EW_ACOS,
 EW_ATAN, EW_ABS, EW_NEG, EW_EXP, EW_LOG, EW_RELU, EW_LEAKY_RELU, EW_SIGMOID, EW_TANH,
 EW_SOFTPLUS) = range(21)
RED_SUM, RED_MAX, RED_MIN, RED_MEAN, RED_ARGMAX, RED_VARIANCE = range(6)
(OPT_ADAMW, OPT_RMSPROP, OPT_ADAGRAD, OPT_NADAM, OPT_RADAM, OPT_ADADELTA, OPT_ADABOUND, OPT_RPROP,
 OPT_LAMB) = range(9)
SCHED_STEP, SCHED_EXPONENTIAL, SCHED_COSINE, SCHED_PLATEAU, SCHED_WARMUP = range(5)

_lib = None


class LibraryMissing(RuntimeError):
    pass


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of every function the C header declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(numrs_hip_[a-z0-9_]+)\s*\(", text)))


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python -m numrs_amd.build` (there is no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
