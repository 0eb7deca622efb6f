"""lucid_decode_noalloc (split partials in the library's static device scratch, no workspace
argument) against lucid_decode (caller workspace), through the C ABI: two calls in a row, the
second with smaller sizes, so that scratch contents left by the first call cannot leak into the
second.  Both run the same kernels on the same inputs, so outputs, the token's V' row and the
appended cache rows must agree exactly."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, Hkv, T_past, D, seed):
    g = torch.Generator().manual_seed(seed)
    s = D ** -0.5
    cap = T_past + 8
    mk = lambda *shape: (torch.randn(*shape, generator=g) * s).to(torch.bfloat16).cuda()  # noqa: E731
    return mk(B, Hq, 1, D), mk(B, Hkv, 1, D), mk(B, Hkv, 1, D), mk(B, Hkv, cap, D), mk(B, Hkv, cap, D)


def _call(lib, fn, q, k, v, kc, vc, T_past, ws=None):
    from lucid_amd import _lib
    B, Hq, _, D = q.shape
    Hkv, cap = kc.shape[1], kc.shape[2]
    o = torch.empty(B, 1, Hq, D, dtype=torch.bfloat16, device="cuda")
    vp_new = torch.empty(B, Hkv, 1, D, dtype=torch.float32, device="cuda")
    args = [_lib.ptr(q), _lib.strides3(q, (0, 1, 2)), _lib.ptr(k), _lib.strides3(k, (0, 1, 2)),
            _lib.ptr(v), _lib.strides3(v, (0, 1, 2)), _lib.ptr(kc), _lib.strides3(kc, (0, 1, 2)),
            _lib.ptr(vc), _lib.strides3(vc, (0, 1, 2)), _lib.ptr(o), _lib.strides3(o, (0, 2, 1)), _lib.ptr(vp_new)]
    if ws is not None:
        args.append(_lib.ptr(ws))
    args += [B, Hq, Hkv, T_past, cap, D, D ** -0.5, 1e-5, _lib.stream_handle(q.device)]
    _lib.check(lib, fn(*args), fn.__name__)
    return o, vp_new


def test_noalloc_decode_matches_workspace_decode():
    from lucid_amd import _lib
    lib = _lib.load()
    for B, Hq, Hkv, T_past, D in [(2, 8, 2, 3000, 128), (1, 4, 2, 700, 64)]:
        print(f"case noalloc decode B={B} Hq={Hq} Hkv={Hkv} T_past={T_past} D={D}", flush=True)
        q, k, v, kc, vc = _inputs(B, Hq, Hkv, T_past, D, seed=T_past + D)
        kc2, vc2 = kc.clone(), vc.clone()
        cap = kc.shape[2]
        ws = torch.empty(max(lib.lucid_decode_workspace_bytes(B, Hq, Hkv, cap, D), 256), dtype=torch.uint8,
                         device="cuda")
        o1, v1 = _call(lib, lib.lucid_decode, q, k, v, kc, vc, T_past, ws)
        o2, v2 = _call(lib, lib.lucid_decode_noalloc, q, k, v, kc2, vc2, T_past)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2)
        assert torch.equal(v1, v2)
        assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
