"""noise_es_gradient_noalloc (the allocation-free variant of noise_es_gradient: its split pair sum
uses a fixed device array instead of a caller workspace) against noise_es_gradient with a torch
workspace, both called through the C ABI: bit-identical gradients on two calls in a row (the step's
largest gradient, then a smaller one), accumulate mode, and a clear error past the fixed size."""
import ctypes as C

import pytest
import torch

from noise_amd import _lib

pytestmark = pytest.mark.gpu


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _case(device, n, out, inn, seed, vector=False):
    g = torch.Generator(device=device).manual_seed(seed)
    buf = torch.randn(1 << 22, device=device, generator=g)
    w = torch.randn(n, device=device, generator=g)
    a_off = torch.randint(0, buf.numel() - out - inn, (n,), device=device, generator=g)
    b_off = None if vector else a_off + out
    return buf, w, a_off, b_off


def _grad_with_workspace(lib, stream, buf, w, a_off, b_off, out, inn, scale, G, accumulate):
    n = w.numel()
    elems = int(lib.noise_es_gradient_work(n, out, inn))
    work = torch.empty(max(elems, 1), device=G.device)
    _lib.check(lib.noise_es_gradient(_ptr(w), n, _ptr(buf), _ptr(a_off), _ptr(buf) if b_off is not None else None,
                                     _ptr(b_off), out, inn, scale, accumulate, _ptr(G), _ptr(work), elems, stream),
               'es_gradient')


def _grad_noalloc(lib, stream, buf, w, a_off, b_off, out, inn, scale, G, accumulate):
    _lib.check(lib.noise_es_gradient_noalloc(_ptr(w), w.numel(), _ptr(buf), _ptr(a_off),
                                             _ptr(buf) if b_off is not None else None, _ptr(b_off), out, inn, scale,
                                             accumulate, _ptr(G), stream), 'es_gradient_noalloc')


def test_es_gradient_noalloc_matches_workspace_entry(device):
    lib = _lib.load()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    cap = int(lib.noise_es_gradient_noalloc_capacity())
    assert cap == 8 << 20
    # The step's largest gradient (1536 pairs over [4096, 512], a 4-way split filling the array),
    # then a smaller one that leaves stale partial tiles of the first call in the array, then a
    # vector parameter, each also in accumulate mode.
    for n, out, inn, vector in ((1536, 4096, 512, False), (300, 512, 512, False), (1536, 8, 1, True)):
        buf, w, a_off, b_off = _case(device, n, out, inn, seed=out + n, vector=vector)
        for accumulate in (0, 1):
            base = torch.randn(out, inn, device=device)
            ref, got = base.clone(), base.clone()
            _grad_with_workspace(lib, stream, buf, w, a_off, b_off, out, inn, -1.0 / n, ref, accumulate)
            _grad_noalloc(lib, stream, buf, w, a_off, b_off, out, inn, -1.0 / n, got, accumulate)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), (n, out, inn, accumulate)


def test_es_gradient_noalloc_rejects_oversize(device):
    lib = _lib.load()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    # 4096 pairs over [2048, 3072] split two ways need 2 x 6.3M floats, beyond the fixed 8M: the call
    # is refused before any launch (the inputs are valid for the shape all the same).
    out, inn = 2048, 3072
    assert int(lib.noise_es_gradient_work(4096, out, inn)) > int(lib.noise_es_gradient_noalloc_capacity())
    buf, w, a_off, b_off = _case(device, 4096, out, inn, seed=3)
    G = torch.zeros(out, inn, device=device)
    with pytest.raises(ValueError, match='beyond the fixed'):
        _grad_noalloc(lib, stream, buf, w, a_off, b_off, out, inn, 1.0, G, 0)
    torch.cuda.synchronize()
    assert not bool(G.any())
