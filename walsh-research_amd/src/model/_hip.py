"""ctypes binding of libwalsh_hip.so (the C ABI declared in include/walsh.h).

The library is loaded from ``walsh-research_amd/lib/`` (built in-tree by
``make -C walsh-research_amd``).  There is no fallback: if the library is
missing or no GPU is present, every hot-path op raises.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_HERE, "..", "..", "lib", "libwalsh_hip.so"))

WALSH_F32 = 0
WALSH_BF16 = 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_I = ctypes.c_int

# name -> (restype, argtypes); mirrors include/walsh.h
SIGNATURES = {
    "walsh_abi_version": (_I, []),
    "walsh_last_error": (ctypes.c_char_p, []),
    "walsh_device_arch": (ctypes.c_char_p, []),
    "walsh_timing_begin": (_I, [_I]),
    "walsh_timing_tag": (None, [_I]),
    "walsh_timing_end": (_I, [_P, _P, _I]),
    "walsh_ternary_gamma": (_I, [_P, _I64, _P, _P]),
    "walsh_ternary_quantize": (_I, [_P, _I64, _I64, _P, _P, _P, _P, _P]),
    "walsh_ternary_unpack": (_I, [_P, _I64, _I64, _P, _P]),
    "walsh_ternary_ste_bwd": (_I, [_P, _P, _I64, _I, _P, _P]),
    "walsh_bitmask_workspace_bytes": (_I64, [_I64]),
    "walsh_ternary_from_bitmask": (_I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P]),
    "walsh_hadamard_weight_bytes": (_I64, [_I64, _I64]),
    "walsh_hadamard_prepare": (_I, [_P, _I64, _I64, _P, _P]),
    "walsh_hadamard_linear_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _I, _P]),
    "walsh_hadamard_linear_ex_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _I, _P]),
    "walsh_hadamard_swiglu_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                       _I, _P]),
    "walsh_hadamard_mlp_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                                    _I, _P]),
    "walsh_fht_fwd": (_I, [_P, _I64, _I64, _I, _P, _I, _P]),
    "walsh_hadamard_linear_rope_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _P, _I64, _I, _P]),
    "walsh_hadamard_linear_multi_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P, _I64, _I64,
                                             _I, _I, _P]),
    "walsh_hadamard_linear_multi_ex_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _I64,
                                                _I64, _I, _I, _P]),
    "walsh_hadamard_dense_weight_bytes": (_I64, [_I64, _I64, _I]),
    "walsh_hadamard_dense_prepare": (_I, [_P, _I64, _I64, _I, _I, _P, _P]),
    "walsh_head_mixer_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _I, _P]),
    "walsh_head_mixer_proj_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64, _I, _P]),
    "walsh_hadamard_pack_transpose": (_I, [_P, _I64, _I64, _P, _P]),
    "walsh_hadamard_bwd_workspace_bytes": (_I64, [_I64, _I64, _I64, _I]),
    "walsh_hadamard_linear_bwd": (_I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64, _P, _P,
                                       _P, _I, _P, _I64, _P]),
    "walsh_hadamard_linear_ex_bwd": (_I, [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P,
                                          _I64, _P, _P, _P, _I, _P, _I64, _P]),
    "walsh_octonion_weight_elems": (_I64, [_I64, _I64]),
    "walsh_octonion_prepare": (_I, [_P, _I64, _I64, _P, _I, _P]),
    "walsh_octonion_linear_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _I, _P]),
    "walsh_octonion_fused_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P]),
    "walsh_octonion_prepare_t": (_I, [_P, _I64, _I64, _P, _P, _I, _P]),
    "walsh_octonion_bwd_fold": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _P]),
    "walsh_octonion_bwd_params_workspace_bytes": (_I64, [_I64, _I64, _I64, _I]),
    "walsh_octonion_bwd_params": (_I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I, _P, _I64, _P]),
    "walsh_decode_attention_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "walsh_decode_attention": (_I, [_P, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_float,
                                    _P, _I64, _I64, _I, _P, _I64, _P]),
    "walsh_decode_attention_static": (_I, [_P, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                           ctypes.c_float, _P, _I64, _I64, _I, _P]),
    "walsh_chanmod_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "walsh_chanmod_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, ctypes.c_float, _P, _I64, _P, _I64, _P,
                               ctypes.c_float, ctypes.c_float, _I, _P, _I64, _P, _I, _P, _I64, _P]),
    "walsh_chanmod_apply": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, ctypes.c_float, ctypes.c_float,
                                 _P, _I64, _I, _P]),
    "walsh_chanmod_bwd": (_I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, ctypes.c_float,
                               ctypes.c_float, _P, _I64, _P, _P, _I, _P, _I64, _P]),
    "walsh_prefill_attention": (_I, [_P, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                     ctypes.c_float, _P, _I64, _I64, _I64, _I, _P]),
    "walsh_sinkhorn_fwd": (_I, [_P, _I64, _I64, _I64, ctypes.c_float, _P, _P]),
    "walsh_sinkhorn_bwd": (_I, [_P, _P, _I64, _I64, _I64, ctypes.c_float, _P, _P]),
    "walsh_mhc_pre_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P, ctypes.c_float, _I64, ctypes.c_float,
                               _P, _P, _P, _P, _I64, _I, _P]),
    "walsh_mhc_post_pre_norm_fwd": (_I, [_P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P,
                                         ctypes.c_float, _I64, ctypes.c_float, _P, _P, _P, _P, _I64, _P,
                                         ctypes.c_float, _I, _P]),
    "walsh_mhc_pre_norm_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P, ctypes.c_float, _I64, ctypes.c_float,
                                    _P, _P, _P, _P, _I64, _P, ctypes.c_float, _I, _P]),
    "walsh_mhc_post_fwd": (_I, [_P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P]),
    "walsh_mhc_aggregate_fwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "walsh_mhc_aggregate_bwd": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "walsh_mhc_post_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "walsh_mhc_pre_wide_workspace": (_I64, [_I64, _I64, _I64]),
    "walsh_mhc_pre_wide_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _F, _I64, _F, _P, _P, _P, _P, _I64, _P, _F,
                                    _P, _I64, _I, _P]),
    "walsh_mhc_post_pre_wide_fwd": (_I, [_P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _F,
                                         _I64, _F, _P, _P, _P, _P, _I64, _P, _F, _P, _I64, _I, _P]),
    "walsh_moe_route_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _I64,
                                 _P, _I64, _I, _I, _P]),
    "walsh_moe_router_wide_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "walsh_moe_router_wide_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _P, _P, _P, _P, _P,
                                       _P, _P, _I64, _P, _I64, _I, _P]),
    "walsh_moe_decode_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    # x ldx M C H w1 w2 E k He gate up down gammas work work_bytes sync probs mask weights idx w count probsum
    # n_part y ldy ydtype stream
    "walsh_moe_decode_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I64, _P,
                                  _P, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _I, _P]),
    "walsh_moe_experts_bwd_workspace_bytes": (_I64, [_I64, _I64]),
    "walsh_moe_experts_bwd": (_I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                                   _P, _P, _P, _P, _P, _I64, _P]),
    "walsh_moe_topk_fwd": (_I, [_P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "walsh_moe_scatter": (_I, [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P]),
    "walsh_moe_experts_fwd": (_I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                   _I, _I, _P]),
    "walsh_moe_ffn_fwd": (_I, [_P, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                               _P, _I64, _I, _I, _P]),
}

_lib = None


class WalshHipError(RuntimeError):
    """A walsh_* entry point returned a non-zero status."""


def lib():
    """Load (once) and return the library handle; raise if it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"libwalsh_hip.so not found at {LIB_PATH}; build it with "
                f"`make -C walsh-research_amd` (or __graft_entry__.build())")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def check(rc: int, name: str) -> None:
    if rc != 0:
        msg = lib().walsh_last_error().decode(errors="replace")
        raise WalshHipError(f"{name} failed with status {rc}: {msg}")


_timer = None


class LaunchTimer:
    """Context manager that times every hot-path kernel launch with the
    kernel's own start/stop timestamps (walsh_timing_begin: the library
    launches through hipExtLaunchKernelGGL with an event pair per launch, on
    the launching stream), labelled with the (kernel, bytes, flops) of the
    entry-point call that made it.  Used by bench.py for the roofline."""

    CAPACITY = 1 << 16

    def __init__(self):
        self.meta = []
        self.records = None

    def __enter__(self):
        global _timer
        check(lib().walsh_timing_begin(self.CAPACITY), "walsh_timing_begin")
        _timer = self
        return self

    def __exit__(self, *exc):
        global _timer
        _timer = None
        self.records = self._collect()

    def _collect(self):
        cap = self.CAPACITY
        tags = (ctypes.c_int * cap)()
        ms = (ctypes.c_float * cap)()
        n = lib().walsh_timing_end(tags, ms, cap)
        if n < 0:
            check(n, "walsh_timing_end")
        return [(tags[i], ms[i]) for i in range(n)]

    def summary(self):
        """{kernel: dict(launches, ms, bytes, flops)}: kernel time summed per
        entry-point call (available after the with-block)."""
        per_call = {}
        for tag, ms in self.records:
            if tag >= 0:
                per_call[tag] = per_call.get(tag, 0.0) + ms
        out = {}
        for tag, ms in per_call.items():
            kname, nbytes, flops = self.meta[tag]
            d = out.setdefault(kname, dict(launches=0, ms=0.0, bytes=0, flops=0))
            d["launches"] += 1
            d["ms"] += ms
            d["bytes"] += nbytes
            d["flops"] += flops
        return out


def call(name: str, *args, kernel: str = None, nbytes: int = 0, flops: int = 0) -> None:
    t = _timer
    if t is not None:
        if kernel is None:
            lib().walsh_timing_tag(-1)
        else:
            lib().walsh_timing_tag(len(t.meta))
            t.meta.append((kernel, int(nbytes), int(flops)))
    check(getattr(lib(), name)(*args), name)


def require_device(t: torch.Tensor, what: str = "tensor") -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what} must be on a GPU (the Walsh hot path has no CPU implementation); "
                           f"got device {t.device}")


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return WALSH_F32
    if dt == torch.bfloat16:
        return WALSH_BF16
    raise TypeError(f"activation dtype {dt} is not supported (float32 or bfloat16)")


_cu = {}


def cu_count(device) -> int:
    """Compute units of ``device`` (cached)."""
    i = torch.device(device).index or 0
    if i not in _cu:
        _cu[i] = torch.cuda.get_device_properties(i).multi_processor_count
    return _cu[i]


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
