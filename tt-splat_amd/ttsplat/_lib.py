"""ctypes binding of libttsplat.so (the C ABI declared in include/ttsplat.h).

The library is loaded after torch so that it binds to the HIP runtime torch already loaded
(both carry the SONAME libamdhip64.so.7): device pointers and streams are shared with torch.
There is no fallback: if the library is missing or the GPU is absent, calls raise.
"""
import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libttsplat.so")

_c_int, _c_float, _vp = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
_c_size, _c_i64, _c_u32 = ctypes.c_size_t, ctypes.c_int64, ctypes.c_uint32

# name -> (restype, argtypes); must match include/ttsplat.h
SIGNATURES = {
    "tts_version": (_c_int, []),
    "tts_strerror": (ctypes.c_char_p, [_c_int]),
    "tts_geom_fwd": (_c_int, [_vp, _c_int, _vp, _c_float, _c_float, _vp, _vp, _vp]),
    "tts_geom_bwd": (_c_int, [_vp, _c_int, _vp, _c_float, _c_float, _vp, _vp, _vp]),
    "tts_bin_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "tts_assign_bins": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                 _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _vp]),
    "tts_assign_bins_noalloc": (_c_int, [_vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                         _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                         _vp]),
    "tts_theta_u_gathered": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_float,
                                      _vp, _vp, _vp, _vp]),
    "tts_tile_order": (_c_int, [_vp, _c_int, _c_int, _vp, _vp]),
    "tts_splat_fwd": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_float,
                               _vp, _vp, _vp, _vp]),
    "tts_splat_fwd_mx": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_float,
                                  _vp, _vp, _vp, _c_int, _vp]),
    "tts_splat_fwd_theta": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                     _vp, _vp]),
    "tts_splat_bwd": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_float,
                               _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tts_splat_fwd_rec": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_float,
                                   _vp, _vp, _vp, _vp]),
    "tts_splat_fwd_mx_rec": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_float,
                                      _vp, _vp, _vp, _c_int, _vp]),
    "tts_splat_bwd_rec": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_float,
                                   _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tts_splat_fwd_theta_bf16": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp,
                                          _vp, _vp, _vp]),
    "tts_splat_bwd_theta_bf16": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp,
                                          _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tts_splat_bwd_theta": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                     _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tts_loss_stats_bytes": (_c_size, [_c_int, _c_int]),
    "tts_loss_workspace_bytes": (_c_size, [_c_int, _c_int]),
    "tts_loss_target_stats": (_c_int, [_vp, _c_int, _c_int, _vp, _vp]),
    "tts_loss_grad_stats": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_float, _vp, _vp, _vp]),
    "tts_composite_random_bg": (_c_int, [_vp, _c_int, _c_int, _vp, _c_int, _c_u32, _vp, _vp,
                                         _vp]),
    "tts_loss_partials_count": (_c_int, [_c_int, _c_int, ctypes.POINTER(_c_int)]),
    "tts_loss_grad": (_c_int, [_vp, _vp, _c_int, _c_int, _c_float, _vp, _vp, _vp, _c_size, _vp]),
    "tts_adam_advance": (_c_int, [_vp, _c_float, _c_float, _vp]),
    "tts_adam": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _vp, _c_float, _c_float, _c_float,
                          _vp]),
    "tts_geom_bwd_adam": (_c_int, [_vp, _c_int, _vp, _c_float, _c_float, _vp, _vp, _vp, _vp, _vp,
                                   _vp, _vp, _c_float, _c_float, _c_float, _vp]),
    "tts_slot_reduce": (_c_int, [_vp, _vp, _c_int, _vp, _vp]),
    "tts_slot_scatter": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _vp, _vp]),
    "tts_zero": (_c_int, [_vp, _c_i64, _vp]),
    "tts_geom_bwd_accum": (_c_int, [_vp, _c_int, _vp, _c_float, _c_float, _vp, _vp, _c_float,
                                    _vp, _vp]),
    "tts_geom_fwd_ex": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _vp, _c_float, _c_float, _vp, _vp,
                                 _vp, _c_float, _c_float, _vp]),
    "tts_geom_fwd_assign_bins": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _vp, _c_float, _c_float,
                                          _vp, _vp, _vp, _c_float, _c_float, _c_int, _c_int,
                                          _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp,
                                          _vp, _vp, _vp, _vp, _vp, _c_size, _vp]),
    "tts_geom_bwd_adam_fwd_count": (_c_int, [_vp, _c_int, _vp, _vp, _c_float, _c_float, _vp, _vp,
                                             _vp, _vp, _vp, _vp, _vp, _c_float, _c_float,
                                             _c_float, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                             _c_int, _c_int, _vp, _c_size, _vp]),
    "tts_assign_bins_counted": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                         _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                         _vp, _vp, _c_float, _c_float, _vp, _c_size, _vp]),
    "tts_geom_bwd_ex": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _vp, _c_float, _c_float,
                                 _vp, _vp, _vp, _vp, _vp]),
    "tts_geom_bwd_adam_ex": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _vp, _vp, _c_int, _vp, _c_float,
                                      _c_float, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_float,
                                      _c_float, _c_float, _c_float, _c_float, _c_float, _c_u32,
                                      _vp]),
    "tts_geom_bwd_accum_ex": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _vp, _c_float, _c_float, _vp,
                                       _vp, _c_float, _vp, _vp, _vp, _vp]),
    "tts_depth_weight_workspace_bytes": (_c_size, [_c_int]),
    "tts_depth_weight_adam": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _c_float, _c_float,
                                       _c_float, _vp, _c_size, _vp]),
    "tts_mcmc_reg_grad": (_c_int, [_vp, _c_int, _c_float, _c_float, _vp, _vp]),
    "tts_sgld_noise": (_c_int, [_vp, _c_int, _vp, _c_float, _c_u32, _vp, _vp]),
    "tts_relocate_workspace_bytes": (_c_size, [_c_int]),
    "tts_relocate": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_float, _c_float, _c_u32,
                              _vp, _vp, _vp, _c_size, _vp]),
    "tts_adam_flat": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _c_float, _c_float, _c_float,
                               _vp]),
    "tts_dense_workspace_bytes": (_c_size, [_c_int, _c_int]),
    "tts_render_dense": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_float, _vp, _vp, _vp, _vp]),
    "tts_render_dense_bwd": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_float, _vp, _vp, _vp, _vp,
                                      _vp, _vp, _vp, _c_size, _vp]),
    "tts_render_dense_arm": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_float, _vp, _c_int, _vp, _vp,
                                      _vp, _vp, _vp]),
    "tts_render_dense_arm_bwd": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_float, _vp, _c_int, _vp,
                                          _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _vp]),
    "tts_wsr_dense": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _vp, _vp, _vp, _vp]),
    "tts_wsr_dense_bwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _vp, _vp, _vp, _vp,
                                   _vp, _vp, _vp, _c_size, _vp]),
}

_lib = None


class TTSError(RuntimeError):
    """A libttsplat entry point returned a non-zero code."""


def load():
    """Load (once) and return the ctypes library handle."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TTSError(f"{LIB_PATH} is missing: build it with tt-splat_amd/ttsplat/build.py "
                           "(or __graft_entry__.build()); there is no CPU fallback")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name, *args):
    """Call entry point `name`; raise TTSError with the library's message on failure."""
    code = getattr(load(), name)(*args)
    if code != 0:
        msg = load().tts_strerror(code).decode()
        raise TTSError(f"{name} failed with code {code}: {msg}")
    return code


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream():
    """The current torch stream as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def require(t, name, dtype, shape=None, device=None):
    """Validate a tensor handed to the library: on a GPU, given dtype, contiguous, shape."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (got {t.device}); the HIP path has no CPU fallback")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    return t
