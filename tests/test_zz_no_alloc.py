"""The no-allocation grad norm, la_grad_norm_clip_noalloc, through the C-ABI.

Its stage-1 partials live in a fixed device array inside the library instead
of a caller workspace.  Checked against la_grad_norm_clip with a caller
workspace on the same inputs, bit for bit (sqnorm, coefficient, norm), on two
calls in a row where the second is smaller than the first, so that partials
the first call left in the shared array must not leak into the second; then an
accumulating call, and the CPU checker's exact sum."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from slideformer_amd import _lib

pytestmark = pytest.mark.gpu

_CODE = {torch.float32: _lib.LA_F32, torch.bfloat16: _lib.LA_BF16, torch.float16: _lib.LA_F16}
_NAME = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def _grads(n, dtype, dev, seed, offset=0):
    gen = torch.Generator().manual_seed(seed)
    full = (torch.randn(n + offset, generator=gen) * 1e-3).to(dtype).to(dev)
    return full[offset:]


def _bits(t):
    return t.cpu().view(torch.int32 if t.element_size() == 4 else torch.int64).numpy().copy()


def _with_workspace(L, g, accumulate, sq0, max_norm, stream):
    dev = g.device
    work = torch.empty(max(1, L.la_grad_sqnorm_workspace(g.numel()) // 8), dtype=torch.float64, device=dev)
    sq = sq0.clone()
    coef = torch.empty(1, dtype=torch.float32, device=dev)
    norm = torch.empty(1, dtype=torch.float32, device=dev)
    rc = L.la_grad_norm_clip(_CODE[g.dtype], g.data_ptr(), g.numel(), work.data_ptr(), work.numel() * 8,
                             sq.data_ptr(), accumulate, max_norm, coef.data_ptr(), norm.data_ptr(), stream)
    assert rc == 0, L.la_strerror(rc)
    torch.cuda.synchronize()
    return sq, coef, norm


def _no_alloc(L, g, accumulate, sq0, max_norm, stream):
    dev = g.device
    sq = sq0.clone()
    coef = torch.empty(1, dtype=torch.float32, device=dev)
    norm = torch.empty(1, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    rc = L.la_grad_norm_clip_noalloc(_CODE[g.dtype], g.data_ptr(), g.numel(), sq.data_ptr(), accumulate,
                                     max_norm, coef.data_ptr(), norm.data_ptr(), stream)
    assert rc == 0, L.la_strerror(rc)
    torch.cuda.synchronize()
    return sq, coef, norm


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_no_alloc_norm_equals_workspace_norm_on_two_calls(dtype, hip_device):
    L = _lib.load()
    stream = torch.cuda.current_stream(hip_device).cuda_stream
    # first call large (every one of the 256 stage-1 workgroups writes a
    # partial), second small and misaligned (one workgroup, head elements)
    sizes = [(20_000_003, 0, 11), (70_001, 1, 12)]
    zero = torch.zeros(1, dtype=torch.float64, device=hip_device)
    for n, offset, seed in sizes:
        print(f"no-alloc norm: dtype {dtype} n {n} offset {offset} seed {seed}", flush=True)
        g = _grads(n, dtype, hip_device, seed, offset)
        ref = _with_workspace(L, g, 0, zero, 1.0, stream)
        got = _no_alloc(L, g, 0, zero, 1.0, stream)
        for a, b, what in zip(got, ref, ("sqnorm", "coef", "norm")):
            assert np.array_equal(_bits(a), _bits(b)), (what, a.item(), b.item())
        # the exact float64 sum of squares of the same values (compensated, CPU)
        exact = O.grad_sqnorm(g.cpu().view(torch.int16 if g.element_size() == 2 else torch.int32).numpy()
                              .view(np.uint16 if g.element_size() == 2 else np.float32).copy(), _NAME[dtype])
        assert abs(got[0].item() - exact) <= 1e-12 * exact
        c_ref, _ = O.clip_coef(exact, 1.0)
        assert got[1].item() == np.float32(c_ref)
        # an accumulating call adds to the caller's running sum, as the workspace call does
        ref_acc = _with_workspace(L, g, 1, ref[0], 0.5, stream)
        got_acc = _no_alloc(L, g, 1, got[0], 0.5, stream)
        for a, b, what in zip(got_acc, ref_acc, ("sqnorm", "coef", "norm")):
            assert np.array_equal(_bits(a), _bits(b)), ("accumulate", what, a.item(), b.item())


def test_no_alloc_norm_on_a_side_stream_and_empty_input(hip_device):
    L = _lib.load()
    side = torch.cuda.Stream(hip_device)
    g = _grads(3_000_017, torch.bfloat16, hip_device, 21)
    zero = torch.zeros(1, dtype=torch.float64, device=hip_device)
    ref = _with_workspace(L, g, 0, zero, 1.0, torch.cuda.current_stream(hip_device).cuda_stream)
    got = _no_alloc(L, g, 0, zero, 1.0, side.cuda_stream)
    for a, b in zip(got, ref):
        assert np.array_equal(_bits(a), _bits(b))
    # n = 0: the sum is 0 and the coefficient 1, as with a workspace
    empty = torch.empty(0, dtype=torch.bfloat16, device=hip_device)
    got0 = _no_alloc(L, empty, 0, zero, 1.0, side.cuda_stream)
    assert got0[0].item() == 0.0 and got0[1].item() == 1.0
    # coef is required
    assert L.la_grad_norm_clip_noalloc(_lib.LA_BF16, g.data_ptr(), g.numel(), zero.data_ptr(), 0, 1.0,
                                       None, None, None) == _lib.LA_EINVAL


def test_no_alloc_norm_checks_the_stream_device(hip_device):
    """The fixed array's address is the current device's, so the stream must
    belong to the current device: the default stream (NULL), the legacy and
    the per-thread default stream and a stream created on the current device
    are accepted,
    with the same bits as the workspace call; a stream of another device is
    refused with LA_EINVAL before any launch (needs a second GPU)."""
    L = _lib.load()
    g = _grads(1_000_003, torch.bfloat16, hip_device, 23)
    zero = torch.zeros(1, dtype=torch.float64, device=hip_device)
    ref = _with_workspace(L, g, 0, zero, 1.0, torch.cuda.current_stream(hip_device).cuda_stream)
    own = torch.cuda.Stream(hip_device)
    for name, st in (("NULL", None), ("legacy", ctypes.c_void_p(1)), ("per-thread", ctypes.c_void_p(2)),
                     ("created", own.cuda_stream)):
        print(f"no-alloc norm on the {name} stream", flush=True)
        got = _no_alloc(L, g, 0, zero, 1.0, st)
        for a, b in zip(got, ref):
            assert np.array_equal(_bits(a), _bits(b)), name
    if torch.cuda.device_count() < 2:
        return
    other = torch.device("cuda", (hip_device.index + 1) % torch.cuda.device_count())
    foreign = torch.cuda.Stream(other)
    sq = zero.clone()
    coef = torch.full((1,), -1.0, device=hip_device)
    torch.cuda.synchronize()
    rc = L.la_grad_norm_clip_noalloc(_lib.LA_BF16, g.data_ptr(), g.numel(), sq.data_ptr(), 0, 1.0,
                                     coef.data_ptr(), None, foreign.cuda_stream)
    assert rc == _lib.LA_EINVAL
    torch.cuda.synchronize()
    assert coef.item() == -1.0 and sq.item() == 0.0
