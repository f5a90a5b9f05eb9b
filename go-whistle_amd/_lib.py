"""ctypes binding of libcqhip.so (include/cqhip.h).

The library is the product: a missing or unloadable libcqhip.so raises
here, loudly; nothing falls back to a CPU path.
"""

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int8, c_int32, c_longlong, c_size_t, c_uint8, c_void_p

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libcqhip.so")

CQ_OK, CQ_ERR_ARG, CQ_ERR_MISUSE, CQ_ERR_DEVICE, CQ_ERR_UNSUPPORTED = 0, 1, 2, 3, 4

# Every symbol include/cqhip.h declares, with (restype, argtypes).
SIGNATURES = {
    "cq_last_error": (c_char_p, []),
    "cq_version": (c_char_p, []),
    "cq_device_info": (c_int, [c_char_p, c_size_t]),
    "cq_new": (c_int, [c_int, c_int, c_int, c_int, c_int, POINTER(c_float), c_size_t, POINTER(c_uint8), c_size_t,
                       POINTER(c_uint8), c_size_t, c_int, POINTER(c_void_p)]),
    "cq_free": (None, [c_void_p]),
    "cq_out": (c_int, [c_void_p]),
    "cq_in": (c_int, [c_void_p]),
    "cq_bits": (c_int, [c_void_p]),
    "cq_prepare": (c_int, [c_void_p]),
    "cq_bytes": (c_longlong, [c_void_p]),
    "cq_device_bytes": (c_longlong, [c_void_p]),
    "cq_rows": (c_int, [c_void_p, c_int, c_int, POINTER(c_void_p)]),
    "cq_exact": (c_int, [c_void_p, POINTER(c_void_p)]),
    "cq_dense": (c_int, [c_void_p, POINTER(c_void_p)]),
    "cq_kernel_name": (c_char_p, [c_void_p]),
    "cq_row": (c_int, [c_void_p, POINTER(c_float), c_size_t, c_int]),
    "cq_gemm": (c_int, [c_void_p, POINTER(c_float), c_size_t, POINTER(c_float), c_size_t, c_int]),
    "cq_gemms": (c_int, [c_int, POINTER(c_void_p), POINTER(POINTER(c_float)), POINTER(c_size_t), POINTER(c_float),
                         c_size_t, c_int]),
    "cq_gemm_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "cq_gemm_mfma_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "cq_gemm_path": (c_char_p, [c_void_p, c_int]),
    "cq_gemms_dev": (c_int, [c_int, POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_int, c_void_p]),
    "cq_workspace_held": (c_longlong, []),
    "kv_attend_int8_paged_dev": (c_int, [c_void_p, c_longlong, c_void_p, c_longlong, c_int, c_int, c_void_p, c_void_p,
                                         c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_float,
                                         c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                         c_void_p]),
    "nd_qkv_prep_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "nd_norm_scaled_add_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int, c_int, c_void_p]),
    "nd_rms_unit_quant_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "nd_expand_lanes_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "nd_collapse_lanes_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "kv_page_copy_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "nd_gather_rows_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_longlong, c_void_p]),
    "cq_workspace_trim": (c_longlong, []),
    "cq_row_dev": (c_int, [c_void_p, c_void_p, c_int, c_void_p]),
    "cq_row_gather_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_float, c_void_p]),
    "cq_batch_new": (c_int, [c_int, POINTER(c_void_p), POINTER(c_void_p), POINTER(c_void_p), POINTER(c_int),
                             POINTER(c_void_p)]),
    "cq_batch_run": (c_int, [c_void_p, c_void_p]),
    "cq_batch_launches": (c_int, [c_void_p]),
    "cq_batch_free": (None, [c_void_p]),
    "kv_quantize_rows": (c_int, [POINTER(c_int8), POINTER(c_float), POINTER(c_float), c_int, c_int, c_int]),
    "kv_quantize_rows_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "kv_attend_int8_dev": (c_int, [c_void_p, c_longlong, c_void_p, c_longlong, c_int, c_int, c_void_p, c_void_p,
                                   c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_longlong, c_longlong, c_void_p,
                                   c_int, c_float, c_int, c_int, c_void_p]),
    "kv_append_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_longlong, c_longlong, c_void_p,
                              c_int, c_void_p]),
    "kv_append_rope_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_longlong, c_longlong,
                                   c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "kv_attend_int8_rope_dev": (c_int, [c_void_p, c_longlong, c_void_p, c_longlong, c_int, c_int, c_void_p, c_void_p,
                                        c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_longlong, c_longlong,
                                        c_void_p, c_int, c_float, c_int, c_int, c_void_p, c_void_p, c_void_p,
                                        c_void_p]),
    "cq_gemms_fused_dev": (c_int, [c_int, POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_int, c_void_p, c_void_p,
                                   c_int, c_void_p]),
    "cq_gemms_append_dev": (c_int, [c_int, POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_int, c_void_p,
                                    POINTER(c_void_p), POINTER(c_void_p), c_longlong, c_longlong, c_void_p, c_int,
                                    POINTER(c_void_p), POINTER(c_void_p), c_void_p]),
    "nd_zcrmsnorm_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "nd_rope_dev": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p]),
    "nd_argmax_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "nd_argmax_advance_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p]),
    "nd_argmax_advance_eos_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p,
                                          c_int, c_void_p]),
    "kv_attend_int8_shared_dev": (c_int, [c_void_p, c_longlong, c_void_p, c_longlong, c_int, c_int, c_void_p,
                                          c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_longlong,
                                          c_longlong, c_void_p, c_int, c_float, c_int, c_int, c_void_p, c_int,
                                          c_void_p]),
    "nd_silu_dev": (c_int, [c_void_p, c_longlong, c_void_p]),
    "nd_fake_quant_dev": (c_int, [c_void_p, c_void_p, c_longlong, c_int, c_int, c_void_p]),
    "kv_reorder_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                               c_void_p]),
    "kv_reorder_noalloc_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                       c_void_p]),
    "nd_add_dev": (c_int, [c_void_p, c_void_p, c_longlong, c_void_p]),
    "nd_sigmoid_gate_dev": (c_int, [c_void_p, c_void_p, c_longlong, c_void_p]),
    "nd_rms_unit_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "nd_mhc_heads_dev": (c_int, [c_void_p] * 8 + [c_int, c_int, c_int, c_void_p, c_void_p]),
    "nd_mhc_heads_stacked_dev": (c_int, [c_void_p] * 6 + [c_int, c_int, c_int, c_void_p, c_void_p]),
    "nd_mhc_mix_dev": (c_int, [c_void_p] * 6 + [c_int, c_int, c_int, c_void_p]),
    "nd_hadamard_mlp_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, POINTER(c_void_p),
                                    POINTER(c_void_p), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "cq_gemms_gated_dev": (c_int, [c_int, POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_void_p, c_int, c_void_p,
                                   c_void_p]),
    "cq_tables_bytes": (c_size_t, [c_int, POINTER(c_void_p), c_int]),
    "cq_gemm_tables_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, POINTER(c_void_p),
                                   c_void_p, c_void_p, c_size_t, POINTER(c_int), c_void_p]),
    "cq_gemms_tables_dev": (c_int, [c_int, POINTER(c_void_p), POINTER(c_void_p), c_int, c_void_p, c_int,
                                    POINTER(c_void_p), POINTER(c_void_p), c_longlong, c_longlong, c_void_p, c_int,
                                    POINTER(c_void_p), POINTER(c_void_p), c_void_p, c_size_t, c_void_p]),
}

_lib = None


def lib():
    """The loaded library with its signatures set; raises if it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libcqhip.so is not built ({LIB_PATH}); run __graft_entry__.build()")
        lb = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(lb, name)
            f.restype = res
            f.argtypes = args
        _lib = lb
    return _lib


class CQError(Exception):
    """A construction error: what the Go API returns as an error value."""


class CQPanic(Exception):
    """Shape misuse: where the Go API panics."""


class CQDeviceError(Exception):
    """A HIP runtime failure or a geometry the library does not run."""


def check(rc):
    if rc == CQ_OK:
        return
    msg = lib().cq_last_error().decode()
    if rc == CQ_ERR_ARG:
        raise CQError(msg)
    if rc == CQ_ERR_MISUSE:
        raise CQPanic(msg)
    raise CQDeviceError(f"{msg} (status {rc})")
