"""ctypes binding of ``libparakeet_paged.so`` (declared in ``include/parakeet_paged.h``).

The library is built in-tree by ``parakeet-streaming_amd/build.py``.  Loading it
never touches the GPU; the kernels run only when a launch entry point is called.
There is no fallback: if the library is missing, :func:`lib` raises.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

LIB_NAME = "libparakeet_paged.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

ABI_VERSION = 9

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

PK_OK = 0
PK_ERR_INVALID = -1
PK_ERR_UNSUPPORTED = -2
PK_ERR_EXHAUSTED = -3
PK_ERR_HIP = -4
PK_ERR_STATE = -5

PCM_S16 = 0
PCM_F32 = 1


class PagedLayout(ctypes.Structure):
    _fields_ = [
        ("k_pool", c_void_p),
        ("v_pool", c_void_p),
        ("num_layers", c_int32),
        ("num_pages", c_int32),
        ("page_size", c_int32),
        ("d_model", c_int32),
        ("rows", c_void_p),
        ("rows_stride", c_int32),
        ("max_pages", c_int32),
    ]


class KvAppendArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32),
        ("device", c_int32),
        ("pages", PagedLayout),
        ("layer", c_int32),
        ("batch", c_int32),
        ("chunk", c_int32),
        ("key", c_void_p),
        ("key_stride_b", c_int64),
        ("key_stride_t", c_int64),
        ("value", c_void_p),
        ("value_stride_b", c_int64),
        ("value_stride_t", c_int64),
    ]


class KvGatherArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32),
        ("device", c_int32),
        ("pages", PagedLayout),
        ("layer", c_int32),
        ("batch", c_int32),
        ("window", c_int32),
        ("end_offset", c_int32),
        ("out_k", c_void_p),
        ("out_k_stride_b", c_int64),
        ("out_k_stride_t", c_int64),
        ("out_v", c_void_p),
        ("out_v_stride_b", c_int64),
        ("out_v_stride_t", c_int64),
    ]


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32),
        ("device", c_int32),
        ("pages", PagedLayout),
        ("layer", c_int32),
        ("batch", c_int32),
        ("chunk", c_int32),
        ("num_heads", c_int32),
        ("head_dim", c_int32),
        ("left", c_int32),
        ("append", c_int32),
        ("query", c_void_p),
        ("query_stride_b", c_int64),
        ("query_stride_t", c_int64),
        ("key", c_void_p),
        ("key_stride_b", c_int64),
        ("key_stride_t", c_int64),
        ("value", c_void_p),
        ("value_stride_b", c_int64),
        ("value_stride_t", c_int64),
        ("pos", c_void_p),
        ("pos_stride", c_int64),
        ("pos_rows", c_int32),
        ("bias_u", c_void_p),
        ("bias_v", c_void_p),
        ("mask", c_void_p),
        ("mask_stride_b", c_int64),
        ("mask_stride_h", c_int64),
        ("mask_stride_t", c_int64),
        ("processed_frames", c_void_p),
        ("cache_lengths", c_void_p),
        ("lengths", c_void_p),
        ("length_scalar", c_int64),
        ("chunk_size", c_int32),
        ("out", c_void_p),
        ("out_stride_b", c_int64),
        ("out_stride_t", c_int64),
        ("rows_per_lane", c_int32),
        ("start_event", c_void_p),
        ("stop_event", c_void_p),
        ("live_streams", c_void_p),
        ("pos_stride_b", c_int64),
    ]


class MaskArgs(ctypes.Structure):
    _fields_ = [
        ("device", c_int32),
        ("batch", c_int32),
        ("chunk", c_int32),
        ("left", c_int32),
        ("chunk_size", c_int32),
        ("processed_frames", c_void_p),
        ("cache_lengths", c_void_p),
        ("lengths", c_void_p),
        ("length_scalar", c_int64),
        ("att_mask", c_void_p),
        ("pad_mask", c_void_p),
    ]


class ConvArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32),
        ("device", c_int32),
        ("batch", c_int32),
        ("chunk", c_int32),
        ("d_model", c_int32),
        ("kernel", c_int32),
        ("glu_in", c_void_p),
        ("glu_in_stride_b", c_int64),
        ("glu_in_stride_t", c_int64),
        ("cache", c_void_p),
        ("num_slots", c_int32),
        ("num_layers", c_int32),
        ("layer", c_int32),
        ("slots", c_void_p),
        ("pad_mask", c_void_p),
        ("lengths", c_void_p),
        ("length_scalar", c_int64),
        ("dw_weight", c_void_p),
        ("dw_bias", c_void_p),
        ("ln_weight", c_void_p),
        ("ln_bias", c_void_p),
        ("ln_eps", ctypes.c_float),
        ("out", c_void_p),
        ("out_stride_b", c_int64),
        ("out_stride_t", c_int64),
    ]


class ResNormArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32),
        ("device", c_int32),
        ("rows", c_int32),
        ("d_model", c_int32),
        ("alpha", ctypes.c_float),
        ("ln_eps", ctypes.c_float),
        ("residual", c_void_p),
        ("residual_stride", c_int64),
        ("branch", c_void_p),
        ("branch_stride", c_int64),
        ("ln_weight", c_void_p),
        ("ln_bias", c_void_p),
        ("residual_out", c_void_p),
        ("residual_out_stride", c_int64),
        ("norm_out", c_void_p),
        ("norm_out_stride", c_int64),
    ]


class FeStream(ctypes.Structure):
    _fields_ = [
        ("slot", c_int32),
        ("n_new", c_int32),
        ("sample_base", c_int64),
        ("frame0", c_int32),
        ("n_frames", c_int32),
        ("noise_id", ctypes.c_uint32),
        ("reserved", c_int32),
    ]


class FeArgs(ctypes.Structure):
    _fields_ = [
        ("device", c_int32),
        ("batch", c_int32),
        ("streams", c_void_p),
        ("pcm_dtype", c_int32),
        ("samples", c_void_p),
        ("samples_stride", c_int64),
        ("sample_ring", c_void_p),
        ("num_slots", c_int32),
        ("ring_size", c_int32),
        ("mel_ring", c_void_p),
        ("mel_ring_rows", c_int32),
        ("n_mels", c_int32),
        ("window", c_void_p),
        ("win_length", c_int32),
        ("n_fft", c_int32),
        ("hop", c_int32),
        ("fb", c_void_p),
        ("fb_range", c_void_p),
        ("preemph", ctypes.c_float),
        ("dither", ctypes.c_float),
        ("seed", ctypes.c_uint64),
        ("log_guard", ctypes.c_float),
        ("max_new", c_int32),
        ("max_frames", c_int32),
    ]


class SubStream(ctypes.Structure):
    _fields_ = [
        ("slot", c_int32),
        ("row0", c_int32),
        ("rows", c_int32),
        ("length", c_int32),
        ("drop", c_int32),
        ("n_out", c_int32),
        ("out_row", c_int32),
        ("reserved", c_int32),
    ]


class SubArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32),
        ("device", c_int32),
        ("batch", c_int32),
        ("streams", c_void_p),
        ("feats", c_void_p),
        ("feat_slots", c_int32),
        ("feat_rows", c_int32),
        ("feat_ring", c_int32),
        ("n_mels", c_int32),
        ("channels", c_int32),
        ("w0", c_void_p),
        ("b0", c_void_p),
        ("w2", c_void_p),
        ("b2", c_void_p),
        ("w3", c_void_p),
        ("b3", c_void_p),
        ("w5", c_void_p),
        ("b5", c_void_p),
        ("w6", c_void_p),
        ("b6", c_void_p),
        ("out", c_void_p),
        ("out_rows", c_int32),
        ("max_out", c_int32),
    ]


class RnntArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32),
        ("device", c_int32),
        ("batch", c_int32),
        ("slots", c_void_p),
        ("num_slots", c_int32),
        ("layers", c_int32),
        ("hidden", c_int32),
        ("joint", c_int32),
        ("vocab1", c_int32),
        ("blank", c_int32),
        ("max_symbols", c_int32),
        ("prime", c_int32),
        ("embed", c_void_p),
        ("w_ih", c_void_p),
        ("w_hh", c_void_p),
        ("b_ih", c_void_p),
        ("b_hh", c_void_p),
        ("w_pred", c_void_p),
        ("b_pred", c_void_p),
        ("w_out", c_void_p),
        ("b_out", c_void_p),
        ("h", c_void_p),
        ("c", c_void_p),
        ("pred_proj", c_void_p),
        ("enc_proj", c_void_p),
        ("enc_stride_b", c_int64),
        ("enc_stride_t", c_int64),
        ("lengths", c_void_p),
        ("max_frames", c_int32),
        ("compact", c_int32),
        ("tokens", c_void_p),
        ("frame_counts", c_void_p),
        ("workspace", c_void_p),
    ]


# name -> (restype, argtypes); exactly the functions include/parakeet_paged.h declares
SIGNATURES = {
    "pk_kv_append": (c_int, [POINTER(KvAppendArgs), c_void_p]),
    "pk_kv_gather": (c_int, [POINTER(KvGatherArgs), c_void_p]),
    "pk_paged_relpos_attn": (c_int, [POINTER(AttnArgs), c_void_p]),
    "pk_streaming_mask": (c_int, [POINTER(MaskArgs), c_void_p]),
    "pk_conv_step": (c_int, [POINTER(ConvArgs), c_void_p]),
    "pk_residual_norm": (c_int, [POINTER(ResNormArgs), c_void_p]),
    "pk_fe_step": (c_int, [POINTER(FeArgs), c_void_p]),
    "pk_subsample": (c_int, [POINTER(SubArgs), c_void_p]),
    "pk_rnnt_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32, c_int32, c_int32]),
    "pk_rnnt_greedy_step": (c_int, [POINTER(RnntArgs), c_void_p]),
    "pk_rnnt_greedy_step_static": (c_int, [POINTER(RnntArgs), c_void_p]),
    "pk_pool_create": (
        c_int,
        [c_int32, c_int32, c_int32, c_int32, c_int32, POINTER(c_int32), POINTER(c_void_p)],
    ),
    "pk_pool_destroy": (None, [c_void_p]),
    "pk_pool_max_pages": (c_int, [c_void_p]),
    "pk_pool_advance": (c_int, [c_void_p, c_int32, POINTER(c_int32), POINTER(c_int32), c_int32]),
    "pk_pool_reset_slot": (c_int, [c_void_p, c_int32]),
    "pk_pool_reset_all": (c_int, [c_void_p]),
    "pk_pool_free_pages": (c_int, [c_void_p]),
    "pk_pool_slot_info": (c_int, [c_void_p, c_int32, POINTER(c_int64), POINTER(c_int32)]),
    "pk_pool_free_list": (c_int, [c_void_p, POINTER(c_int32), c_int32]),
    "pk_hbm_read_probe": (c_int, [c_void_p, c_int64, c_void_p, c_int32, c_void_p, c_void_p, c_void_p]),
    "pk_last_error": (c_char_p, []),
    "pk_abi_version": (c_int, []),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Loads the library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with parakeet-streaming_amd/build.py "
                    "(the paged KV-cache path has no non-HIP fallback)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            version = handle.pk_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH}: ABI version {version}, expected {ABI_VERSION}")
            _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().pk_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> int:
    """Raises RuntimeError for a negative return code (the reference raises
    RuntimeError for unusable state, parakeet/engine/scheduler.py:112,132)."""
    if rc < 0:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")
    return rc
