"""The C-ABI libraries load on the CPU and export every symbol their headers declare.

No compute call is made here (there is no GPU in the CPU suite): only pure host
functions (ABI version, workspace sizes, argument validation that rejects a
call before anything is launched) are exercised.
"""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))
LIB_FOR_HEADER = {"lucid_amd.h": "liblucid_amd.so", "lucid_path.h": "liblucid_path.so"}


def _declared(header):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(lucid\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def built():
    """Use the in-tree libraries; build only those that are missing (build() is the driver's job)."""
    from lucid_amd import _lib, build
    if not all(os.path.exists(_lib.lib_path(n)) for n in build.TARGETS):
        build.build()
    return True


@pytest.mark.parametrize("header", HEADERS, ids=os.path.basename)
def test_every_declared_symbol_is_exported(built, header):
    from lucid_amd import _lib
    libname = LIB_FOR_HEADER[os.path.basename(header)]
    lib = _lib.load(libname)
    names = _declared(header)
    assert names, "no declarations parsed"
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{libname} lacks {missing}"


def test_abi_version_and_workspace(built):
    from lucid_amd import _lib
    lib = _lib.load()
    assert lib.lucid_abi_version() == 6
    ws = lib.lucid_fwd_workspace_bytes(1, 16, 16, 32768, 64)
    # rinv + K^T + K^ (bf16) + V' (bf16) + V'^T + diagonal inverses + -(X_B P_BA) per 128-row
    # block + lo parts of V' and V'^T + row masses + lo part of O + counters, each 256-byte aligned
    expect = (16 * 32768 * 4 + 4 * 16 * 64 * 32768 * 2 + 16 * 512 * 4096 * 4 + 16 * 256 * 4096 * 4
              + 2 * 16 * 64 * 32768 * 2 + 256 + 16 * 32768 * 64 * 2 + 256)
    assert ws == expect
    assert lib.lucid_fwd_workspace_mass_offset(1, 16, 16, 32768, 64) == expect - 512 - 16 * 32768 * 64 * 2
    assert lib.lucid_bwd_workspace_bytes(1, 16, 16, 32768, 64) > 0


def test_precision_mode_roundtrip_and_validation(built):
    from lucid_amd import _lib
    lib = _lib.load()
    assert lib.lucid_get_precision() == 0
    for mode in (2, 1, 0):
        assert lib.lucid_set_precision(mode) == 0 and lib.lucid_get_precision() == mode
    assert lib.lucid_set_precision(7) == _lib.LUCID_EINVAL
    assert b"precision" in lib.lucid_last_error() and lib.lucid_get_precision() == 0


def test_decoder_layer_and_optimizer_validation_without_gpu(built):
    """The fused decoder layers and the AdamW step reject bad shapes, pointers and
    hyper-parameters before anything is launched."""
    from lucid_amd import _lib
    lib = _lib.load()
    dummy = ctypes.c_void_p(1 << 20)
    rc = lib.lucid_rmsnorm_fwd(dummy, dummy, dummy, dummy, 4, 768, 1e-5, None)
    assert rc == _lib.LUCID_EINVAL and b"H must be" in lib.lucid_last_error()
    s = (ctypes.c_int64 * 3)(64, 64, 64)
    rc = lib.lucid_rope(dummy, s, 1, 1, 1, dummy, dummy, dummy, s, 128, 0, None)
    assert rc == _lib.LUCID_EINVAL and b"head dim 64" in lib.lucid_last_error()
    odd = (ctypes.c_int64 * 3)(68, 68, 68)
    rc = lib.lucid_rope(dummy, odd, 1, 1, 1, dummy, dummy, dummy, s, 64, 0, None)
    assert rc == _lib.LUCID_EINVAL and b"multiples of 8" in lib.lucid_last_error()
    rc = lib.lucid_rope(dummy, s, 1, 1, 1, dummy, dummy, dummy, odd, 64, 0, None)
    assert rc == _lib.LUCID_EINVAL and b"multiples of 8" in lib.lucid_last_error()
    rc = lib.lucid_swiglu_fwd(ctypes.c_void_p((1 << 20) + 2), dummy, dummy, 64, None)
    assert rc == _lib.LUCID_EINVAL and b"aligned" in lib.lucid_last_error()
    rc = lib.lucid_causal_lm_loss_fwd(dummy, 100, dummy, 4, 4, 100, dummy, dummy, dummy, None)
    assert rc == _lib.LUCID_EINVAL and b"multiples of 8" in lib.lucid_last_error()
    rc = lib.lucid_causal_lm_loss_fwd(dummy, 64, dummy, 6, 4, 64, dummy, dummy, dummy, None)
    assert rc == _lib.LUCID_EINVAL and b"multiple of T" in lib.lucid_last_error()

    def adamw(ptr, numel, dtype=0, beta2=0.999, step=1):
        arrs = [(ctypes.c_void_p * 1)(ptr) for _ in range(4)]
        return lib.lucid_adamw_step(1, *arrs, (ctypes.c_int64 * 1)(numel), dtype, 1e-3, 0.9, beta2, 1e-8, 0.01,
                                    step, None)
    assert adamw(1 << 20, 8, dtype=2) == _lib.LUCID_EINVAL
    assert adamw(1 << 20, 8, step=0) == _lib.LUCID_EINVAL
    assert adamw(1 << 20, 8, beta2=1.0) == _lib.LUCID_EINVAL and b"betas" in lib.lucid_last_error()
    assert adamw((1 << 20) + 16, 8, dtype=1) == _lib.LUCID_EINVAL and b"aligned" in lib.lucid_last_error()
    assert adamw(1 << 20, -1) == _lib.LUCID_EINVAL and b"element count" in lib.lucid_last_error()
    assert lib.lucid_adamw_step(0, None, None, None, None, None, 0, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, None) == 0


def test_argument_validation_without_gpu(built):
    from lucid_amd import _lib
    lib = _lib.load()
    s = (ctypes.c_int64 * 3)(64 * 256, 64 * 256, 64)
    dummy = ctypes.c_void_p(1 << 20)
    # head dims above 128 (or below 1) are rejected before anything is launched
    for d in (0, 129, 256):
        rc = lib.lucid_attn_fwd(dummy, s, dummy, s, dummy, s, dummy, s, dummy, dummy, dummy,
                                1, 1, 1, 256, d, 0.1, 1e-5, None)
        assert rc == _lib.LUCID_EINVAL
        assert b"head_dim" in lib.lucid_last_error()
    # other head dims run on rows padded to 64 or 128: the workspaces are those of the padded dim
    for d, dp in ((1, 64), (32, 64), (68, 128), (96, 128)):
        assert lib.lucid_fwd_workspace_bytes(1, 4, 2, 256, d) == lib.lucid_fwd_workspace_bytes(1, 4, 2, 256, dp)
        assert lib.lucid_bwd_workspace_bytes(1, 4, 2, 256, d) == lib.lucid_bwd_workspace_bytes(1, 4, 2, 256, dp)
        assert lib.lucid_decode_workspace_bytes(1, 4, 2, 4096, d) == lib.lucid_decode_workspace_bytes(1, 4, 2, 4096, dp)
    # fp32 inputs: head dims up to 128 as well (workspaces of the padded dim), above rejected
    rc = lib.lucid_attn_fwd_f32(dummy, s, dummy, s, dummy, s, dummy, s, dummy, dummy, dummy,
                                1, 1, 1, 256, 129, 0.1, 1e-5, None)
    assert rc == _lib.LUCID_EINVAL and b"head_dim" in lib.lucid_last_error()
    assert lib.lucid_fwd_f32_workspace_bytes(1, 4, 2, 256, 68) == lib.lucid_fwd_f32_workspace_bytes(1, 4, 2, 256, 128)
    rc = lib.lucid_attn_fwd(dummy, s, dummy, s, dummy, s, dummy, s, dummy, dummy, dummy,
                            1, 1, 1, 200, 64, 0.1, 1e-5, None)
    assert rc == _lib.LUCID_EINVAL and b"multiple of 128" in lib.lucid_last_error()
    rc = lib.lucid_attn_fwd(dummy, s, dummy, s, dummy, s, dummy, s, dummy, dummy, dummy,
                            1, 3, 2, 256, 64, 0.1, 1e-5, None)
    assert rc == _lib.LUCID_EINVAL and b"multiple of Hkv" in lib.lucid_last_error()
    # workspaces must be 256-byte aligned (chain blocks fill whole cache lines)
    misaligned = ctypes.c_void_p((1 << 20) + 128)
    rc = lib.lucid_attn_fwd(dummy, s, dummy, s, dummy, s, dummy, s, dummy, dummy, misaligned,
                            1, 1, 1, 256, 64, 0.1, 1e-5, None)
    assert rc == _lib.LUCID_EINVAL and b"256-byte aligned" in lib.lucid_last_error()
    plib = _lib.load("liblucid_path.so")
    s4 = (ctypes.c_int64 * 3)(64 * 256, 64, 64)
    sb = (ctypes.c_int64 * 3)(256, 1, 1)
    rc = plib.lucid_path_fwd(dummy, s4, dummy, s4, dummy, s4, dummy, s4, dummy, sb, dummy, s4, None, None,
                             misaligned, 1, 256, 1, 1, 64, 0.125, None)
    assert rc == _lib.LUCID_EINVAL and b"256-byte aligned" in plib.lucid_path_last_error()
    rc = plib.lucid_path_softmax_fwd(dummy, s4, dummy, s4, dummy, s4, dummy, s4, dummy, sb, dummy, s4, None, None,
                                     misaligned, 1, 256, 1, 1, 64, 0.125, None)
    assert rc == _lib.LUCID_EINVAL and b"256-byte aligned" in plib.lucid_path_last_error()
    # the path kernels run at head dims 64 and 128 (the Python layer pads the others)
    rc = plib.lucid_path_softmax_fwd(dummy, s4, dummy, s4, dummy, s4, dummy, s4, dummy, sb, dummy, s4, None, None,
                                     dummy, 1, 256, 1, 1, 96, 0.125, None)
    assert rc == _lib.LUCID_EINVAL and b"head_dim" in plib.lucid_path_last_error()
    # fp32: head dim 64 only; its workspaces add the lo planes of the bf16 operand copies
    rc = plib.lucid_path_fwd_f32(dummy, s4, dummy, s4, dummy, s4, dummy, s4, dummy, sb, dummy, s4, None, None,
                                 dummy, 1, 256, 1, 1, 128, 0.125, None)
    assert rc == _lib.LUCID_EINVAL and b"fp32" in plib.lucid_path_last_error()
    for kind in ("fwd", "bwd", "softmax_fwd", "softmax_bwd"):
        n16 = getattr(plib, f"lucid_path_{kind}_workspace_bytes")(1, 4096, 2, 4, 64)
        n32 = getattr(plib, f"lucid_path_{kind}_f32_workspace_bytes")(1, 4096, 2, 4, 64)
        assert n32 > n16, kind
    # head dim 128: the KD x KD transport matrices and 128-wide rows
    assert plib.lucid_path_fwd_workspace_bytes(1, 4096, 2, 4, 128) > 2 * plib.lucid_path_fwd_workspace_bytes(1, 4096, 2, 4, 64)
    # the softmax forward workspace drops the solve's inverses and O^T and adds the row lse
    B, T, H, HQ = 1, 4096, 2, 4
    d = plib.lucid_path_fwd_workspace_bytes(B, T, H, HQ, 64) - plib.lucid_path_softmax_fwd_workspace_bytes(B, T, H, HQ, 64)
    assert d == B * HQ * (T // 64) * 4096 * 4 + B * HQ * T * 64 * 2 - B * HQ * T * 4


def test_noalloc_decode_rejects_sizes_beyond_its_scratch_without_gpu(built):
    """lucid_decode_noalloc checks the size of its partials against its 4 MiB static scratch
    before any GPU call: 2048 kv heads of head dim 128 with 8 query heads each need more."""
    from lucid_amd import _lib
    lib = _lib.load()
    dummy = ctypes.c_void_p(1 << 20)
    s = (ctypes.c_int64 * 3)(64 * 256, 64 * 256, 128)
    rc = lib.lucid_decode_noalloc(dummy, s, dummy, s, dummy, s, dummy, s, dummy, s, dummy, s, dummy,
                                  1, 8 * 2048, 2048, 100, 256, 128, 0.088, 1e-5, None)
    assert rc == _lib.LUCID_EINVAL
    assert b"static scratch" in lib.lucid_last_error()


def test_chain_wait_limit_validation_without_gpu(built):
    from lucid_amd import _lib
    lib = _lib.load()
    assert lib.lucid_set_chain_wait_limit(0.0) == _lib.LUCID_EINVAL
    assert b"positive" in lib.lucid_last_error()
    plib = _lib.load("liblucid_path.so")
    assert plib.lucid_path_set_chain_wait_limit(-1.0) == _lib.LUCID_EINVAL


def test_product_path_fails_loudly_without_gpu_tensors():
    import torch
    from lucid_amd import lucid_attention
    q = torch.zeros(1, 1, 128, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        lucid_attention(q, q, q)


def test_tril_solver_asserts_like_the_reference():
    """Lucid_Tril_Solver.forward asserts T > BS and T % BS == 0 (modeling_lucid.py:287-288)
    before anything else, so these raise on the CPU as in the reference."""
    import torch
    from lucid_amd.lucid import Lucid_Tril_Solver
    k = torch.zeros(1, 1, 4096, 64, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="greater than block size"):
        Lucid_Tril_Solver.apply(k, k, 0.125)  # default BS = 2**14
    with pytest.raises(AssertionError, match="divisible by block size"):
        Lucid_Tril_Solver.apply(k, k, 0.125, 3000)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        Lucid_Tril_Solver.apply(k, k, 0.125, 1024)


def test_only_the_declared_entry_points_are_exported(built):
    """Each library exports the extern "C" entry points its header declares and no internal host
    helper: chain_guard (the bounded-wait flag and its per-device set-up) and lucid_prof (event
    records) stay hidden, so two libraries in one process, loaded RTLD_GLOBAL or linked, never
    bind each other's copies or their static state.  What else is visible is the HIP kernel
    handles (namespace lucid, names distinct between the two libraries), libstdc++'s own template
    instances (namespace std, stateless) and HIP's module marker."""
    import subprocess
    from lucid_amd import _lib
    kernels = {}
    for header in HEADERS:
        libname = LIB_FOR_HEADER[os.path.basename(header)]
        out = subprocess.run(["nm", "-D", "--defined-only", _lib.lib_path(libname)], capture_output=True,
                             text=True, check=True).stdout
        names = {ln.split()[-1] for ln in out.splitlines() if len(ln.split()) == 3}
        plain = sorted(n for n in names if not n.startswith("_Z") and not n.startswith("__hip_cuid_"))
        assert plain == _declared(header), f"{libname}: {set(plain) ^ set(_declared(header))}"
        mangled = {n for n in names if n.startswith("_Z")}
        stray = sorted(n for n in mangled if not n.startswith(("_ZN5lucid", "_ZNSt", "_ZSt")))
        assert not stray, f"{libname} exports internal helpers {stray}"
        assert not any("11chain_guard" in n or "10lucid_prof" in n for n in names)
        kernels[libname] = {n for n in mangled if n.startswith("_ZN5lucid")}
    a, b = kernels.values()
    assert not (a & b), f"kernel handles exported by both libraries: {sorted(a & b)}"
