"""ctypes binding of ``liblucid_amd.so`` (C ABI declared in include/lucid_amd.h).

The library is loaded after ``torch`` so that it shares torch's HIP runtime.
There is no fallback: if the library is missing or a call fails, an exception
is raised.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library links against)

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBS: dict[str, ctypes.CDLL] = {}

LUCID_EINVAL = 1
LUCID_ECHAIN = 2
LUCID_EHIP = 1000

_vp = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)
_int = ctypes.c_int
_flt = ctypes.c_float
_sz = ctypes.c_size_t

_SIGS = {
    "liblucid_amd.so": {
        "lucid_abi_version": ([], _int),
        "lucid_last_error": ([], ctypes.c_char_p),
        "lucid_fwd_workspace_bytes": ([_int] * 5, _sz),
        "lucid_set_precision": ([_int], _int),
        "lucid_chain_status": ([], _int),
        "lucid_set_chain_wait_limit": ([ctypes.c_double], _int),
        "lucid_get_precision": ([], _int),
        "lucid_set_fused_forward": ([_int], _int),
        "lucid_get_fused_forward": ([], _int),
        "lucid_fwd_workspace_mass_offset": ([_int] * 5, _sz),
        "lucid_bwd_workspace_bytes": ([_int] * 5, _sz),
        "lucid_get_v_prime": ([_vp, _i64p, _vp, _i64p, _vp, _vp, _int, _int, _int, _int, _flt, _flt, _vp], _int),
        "lucid_attn_fwd": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp, _vp,
                            _int, _int, _int, _int, _int, _flt, _flt, _vp], _int),
        "lucid_attn_bwd": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp,
                            _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                            _int, _int, _int, _int, _int, _flt, _flt, _vp], _int),
        "lucid_fwd_f32_workspace_bytes": ([_int] * 5, _sz),
        "lucid_bwd_f32_workspace_bytes": ([_int] * 5, _sz),
        "lucid_attn_fwd_f32": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp, _vp,
                                _int, _int, _int, _int, _int, _flt, _flt, _vp], _int),
        "lucid_attn_bwd_f32": ([_vp, _i64p, _vp, _i64p, _vp, _vp, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                                _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_v_prime_f32_workspace_bytes": ([_int] * 4, _sz),
        "lucid_get_v_prime_f32": ([_vp, _i64p, _vp, _i64p, _vp, _vp, _int, _int, _int, _int, _flt, _flt, _vp], _int),
        "lucid_precond_bwd_f32": ([_vp, _i64p, _vp, _vp, _i64p, _vp, _i64p, _vp, _int, _int, _int, _int, _flt, _vp],
                                  _int),
        "lucid_attn_vp_fwd_f32_workspace_bytes": ([_int] * 5, _sz),
        "lucid_attn_vp_fwd_f32": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp,
                                   _int, _int, _int, _int, _int, _flt, _flt, _vp], _int),
        "lucid_attn_vp_bwd_f32_workspace_bytes": ([_int] * 5, _sz),
        "lucid_attn_vp_bwd_f32": ([_vp, _i64p, _vp, _i64p, _vp, _vp, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                                   _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_attn_vp_fwd_workspace_bytes": ([_int] * 5, _sz),
        "lucid_attn_vp_fwd": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _int, _vp, _i64p, _vp, _vp,
                               _int, _int, _int, _int, _int, _flt, _flt, _vp], _int),
        "lucid_attn_vp_bwd_workspace_bytes": ([_int] * 5, _sz),
        "lucid_attn_vp_bwd": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp,
                               _vp, _i64p, _vp, _i64p, _vp, _i64p, _int, _vp,
                               _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_precond_bwd_workspace_bytes": ([_int] * 4, _sz),
        "lucid_precond_bwd": ([_vp, _i64p, _vp, _i64p, _int, _vp, _vp, _i64p, _vp, _i64p, _vp,
                               _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_tril_solve": ([_vp, _i64p, _vp, _i64p, _vp, _vp, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_tril_solve_bwd": ([_vp, _i64p, _vp, _i64p, _int, _vp, _vp, _i64p, _vp, _i64p, _vp,
                                  _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_tril_solve_f32": ([_vp, _i64p, _vp, _i64p, _vp, _vp, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_tril_solve_bwd_f32": ([_vp, _i64p, _vp, _vp, _i64p, _vp, _i64p, _vp, _int, _int, _int, _int, _flt,
                                      _vp], _int),
        "lucid_decode_workspace_bytes": ([_int] * 5, _sz),
        "lucid_decode": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp,
                          _int, _int, _int, _int, _int, _int, _flt, _flt, _vp], _int),
        "lucid_decode_noalloc": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                                  _int, _int, _int, _int, _int, _int, _flt, _flt, _vp], _int),
        "lucid_decode_tokens_workspace_bytes": ([_int] * 6, _sz),
        "lucid_rmsnorm_fwd": ([_vp, _vp, _vp, _vp, _int, _int, _flt, _vp], _int),
        "lucid_rmsnorm_bwd_workspace_bytes": ([_int, _int], _sz),
        "lucid_rmsnorm_bwd": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _int, _int, _vp], _int),
        "lucid_rope": ([_vp, _vp, _int, _int, _int, _vp, _vp, _vp, _vp, _int, _int, _vp], _int),
        "lucid_swiglu_fwd": ([_vp, _vp, _vp, ctypes.c_int64, _vp], _int),
        "lucid_swiglu_bwd": ([_vp, _vp, _vp, _vp, _vp, ctypes.c_int64, _vp], _int),
        "lucid_causal_lm_loss_fwd": ([_vp, ctypes.c_int64, _vp, _int, _int, _int, _vp, _vp, _vp, _vp], _int),
        "lucid_causal_lm_loss_bwd": ([_vp, ctypes.c_int64, _vp, _int, _int, _int, _vp, _vp, _vp, _vp, _vp], _int),
        "lucid_adamw_step": ([_int, _vp, _vp, _vp, _vp, _i64p, _int, _flt, _flt, _flt, _flt, _flt, ctypes.c_int64,
                              _vp], _int),
        "lucid_decode_tokens": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp,
                                 _int, _int, _int, _int, _int, _int, _int, _flt, _flt, _vp], _int),
        "lucid_profile_enable": ([_int], None),
        "lucid_profile_collect": ([], _int),
        "lucid_profile_entry": ([_int, ctypes.c_char_p, _int, ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(ctypes.c_long)], _int),
        "lucid_profile_reset": ([], None),
        "lucid_profile_only": ([ctypes.c_char_p], None),
    },
    "liblucid_path.so": {
        "lucid_path_abi_version": ([], _int),
        "lucid_path_last_error": ([], ctypes.c_char_p),
        "lucid_path_chain_status": ([], _int),
        "lucid_path_set_chain_wait_limit": ([ctypes.c_double], _int),
        "lucid_path_fwd_workspace_bytes": ([_int] * 5, _sz),
        "lucid_path_fwd": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                            _vp, _i64p, _vp, _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_path_bwd_workspace_bytes": ([_int] * 5, _sz),
        "lucid_path_bwd": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                            _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                            _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_path_softmax_fwd_workspace_bytes": ([_int] * 5, _sz),
        "lucid_path_softmax_fwd": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                                    _vp, _i64p, _vp, _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_path_softmax_bwd_workspace_bytes": ([_int] * 5, _sz),
        "lucid_path_softmax_bwd": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                                    _vp, _i64p, _vp, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                                    _vp, _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_path_fwd_f32_workspace_bytes": ([_int] * 5, _sz),
        "lucid_path_fwd_f32": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                                _vp, _i64p, _vp, _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_path_bwd_f32_workspace_bytes": ([_int] * 5, _sz),
        "lucid_path_bwd_f32": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                                _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                                _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_path_softmax_fwd_f32_workspace_bytes": ([_int] * 5, _sz),
        "lucid_path_softmax_fwd_f32": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                                        _vp, _i64p, _vp, _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_path_softmax_bwd_f32_workspace_bytes": ([_int] * 5, _sz),
        "lucid_path_softmax_bwd_f32": ([_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                                        _vp, _i64p, _vp, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                                        _i64p, _vp, _int, _int, _int, _int, _int, _flt, _vp], _int),
        "lucid_path_profile_enable": ([_int], None),
        "lucid_path_profile_collect": ([], _int),
        "lucid_path_profile_entry": ([_int, ctypes.c_char_p, _int, ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_long)], _int),
        "lucid_path_profile_reset": ([], None),
        "lucid_path_profile_only": ([ctypes.c_char_p], None),
    },
}


def profile_totals(lib: ctypes.CDLL, prefix: str = "lucid_") -> dict[str, tuple[float, int]]:
    """Collect the per-kernel event timings recorded so far: {name: (total_ms, launches)}.

    ``prefix`` selects the library's profile API ("lucid_" or "lucid_path_")."""
    n = getattr(lib, prefix + "profile_collect")()
    if n < 0:
        raise RuntimeError("profile collect failed")
    out = {}
    buf = ctypes.create_string_buffer(128)
    entry = getattr(lib, prefix + "profile_entry")
    for i in range(n):
        ms, cnt = ctypes.c_double(), ctypes.c_long()
        if entry(i, buf, 128, ctypes.byref(ms), ctypes.byref(cnt)) == 0:
            out[buf.value.decode()] = (ms.value, cnt.value)
    return out


def lib_path(name: str = "liblucid_amd.so") -> str:
    return os.path.join(_HERE, name)


def load(name: str = "liblucid_amd.so") -> ctypes.CDLL:
    """Load (once) and return the named HIP library; raises if it was not built."""
    if name in _LIBS:
        return _LIBS[name]
    path = lib_path(name)
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `python -m lucid_amd.build` "
                           "(there is no CPU fallback)")
    lib = ctypes.CDLL(path)
    for fn, (args, res) in _SIGS[name].items():
        f = getattr(lib, fn)
        f.argtypes = args
        f.restype = res
    _LIBS[name] = lib
    return lib


def chain_status(synchronize: bool = True) -> None:
    """Raise RuntimeError if a chain wait of either library gave up (no progress within the
    wait bound) in a launch since the last check; ``synchronize`` first waits for the
    launches in flight so that they are covered."""
    if synchronize:
        torch.cuda.synchronize()
    for name, fn in (("liblucid_amd.so", "lucid_chain_status"), ("liblucid_path.so", "lucid_path_chain_status")):
        lib = load(name)
        check(lib, getattr(lib, fn)(), fn)


def check(lib: ctypes.CDLL, rc: int, what: str) -> None:
    if rc == 0:
        return
    getter = getattr(lib, "lucid_last_error", None) or getattr(lib, "lucid_path_last_error", None)
    msg = getter().decode(errors="replace") if getter else ""
    if rc == LUCID_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def strides3(t: torch.Tensor, dims: tuple[int, int, int]):
    """Element strides of three axes of ``t`` as a ctypes int64[3]."""
    arr = (ctypes.c_int64 * 3)(*(t.stride(d) for d in dims))
    return arr


def ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def stream_handle(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
