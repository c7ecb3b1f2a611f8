"""The allocation-free graft AdamW step (glt_adamw_graft_step_noalloc),
called through the C ABI, against the workspace form glt_adamw_graft_step on
identical state: masters, moments and the packed bf16 mirrors bit for bit,
over two calls in a row (the second smaller, with a tighter clip, so its
clip reads fewer partial sums than the first left in the library's array)."""
import ctypes

import numpy as np
import pytest

from helpers import draw

pytestmark = pytest.mark.gpu


def _state(torch, ops, shapes, seed):
    slices, grads, ms, vs = [], [], [], []
    for j, (S, H) in enumerate(shapes):
        masters = [torch.from_numpy(draw((S, H), seed + j, p, 0, 0.02, bf16=False)).cuda() for p in range(3)]
        slices.append(ops.GraftSlice(0, S, 0, H, *masters).pack())
        grads.append(torch.from_numpy(draw((3 * S * H,), seed + 10 + j, 1, 0, 0.05, bf16=False)).cuda())
        ms.append(torch.from_numpy(draw((3 * S * H,), seed + 20 + j, 1, 0, 1e-3, bf16=False)).cuda())
        vs.append(torch.from_numpy(np.abs(draw((3 * S * H,), seed + 30 + j, 1, 0, 1e-4, bf16=False))).cuda())
    return slices, grads, ms, vs


def _clone(torch, ops, st):
    slices, grads, ms, vs = st
    out = []
    for sl in slices:
        c = ops.GraftSlice(sl.i_start, sl.s, sl.h_start, sl.h, sl.gate.clone(), sl.up.clone(), sl.down.clone())
        c.packed.copy_(sl.packed)
        out.append(c)
    return out, [g.clone() for g in grads], [t.clone() for t in ms], [t.clone() for t in vs]


def _call(F, ops, name, st, step, clip, extra):
    slices, grads, ms, vs = st
    arr = ops._slices_array(slices)
    F.call(name, arr, len(slices), F.ptr_array([g.data_ptr() for g in grads]), F.ptr_array([t.data_ptr() for t in ms]),
           F.ptr_array([t.data_ptr() for t in vs]), F.ptr_array([s.packed.data_ptr() for s in slices]), 7, step,
           1e-3, 0.9, 0.999, 1e-8, 0.01, clip, *extra, ops._stream())


def test_noalloc_graft_step_matches_workspace_form(dev):
    import torch
    from glt_amd import _ffi as F
    from glt_amd import ops
    ws_bytes = F.load().glt_adamw_workspace_size(0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    for shapes, seed, step, clip in (([(128, 256), (64, 96)], 40, 3, 1.0),   # fused tiles + separate passes
                                     ([(64, 128)], 60, 4, 0.25)):              # smaller, tighter clip
        print("noalloc call", shapes, clip, flush=True)
        a = _state(torch, ops, shapes, seed)
        b = _clone(torch, ops, a)
        _call(F, ops, "glt_adamw_graft_step", a, step, clip, (ctypes.c_void_p(ws.data_ptr()), ws_bytes))
        _call(F, ops, "glt_adamw_graft_step_noalloc", b, step, clip, ())
        torch.cuda.synchronize()
        bits = lambda t: t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)
        for sa, sb in zip(a[0], b[0]):
            for x, y in ((sa.gate, sb.gate), (sa.up, sb.up), (sa.down, sb.down), (sa.packed, sb.packed)):
                assert torch.equal(bits(x), bits(y))
        for xs, ys in ((a[2], b[2]), (a[3], b[3])):
            for x, y in zip(xs, ys):
                assert torch.equal(bits(x), bits(y))
        # the clip acted (the moments differ from an unclipped step)
        c = _clone(torch, ops, _state(torch, ops, shapes, seed))
        _call(F, ops, "glt_adamw_graft_step", c, step, 0.0, (None, 0))
        torch.cuda.synchronize()
        assert not torch.equal(c[2][0], b[2][0])


def test_noalloc_graft_step_many_slices(dev):
    """More slices than one launch of the clip or of the fused update takes
    (12 slices, 36 projections, one clip norm over all of them): the
    allocation-free form against the workspace form bit for bit."""
    import torch
    from glt_amd import _ffi as F
    from glt_amd import ops
    ws_bytes = F.load().glt_adamw_workspace_size(0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    shapes = [(64, 128)] * 11 + [(64, 96)]
    a = _state(torch, ops, shapes, 80)
    b = _clone(torch, ops, a)
    _call(F, ops, "glt_adamw_graft_step", a, 2, 1.0, (ctypes.c_void_p(ws.data_ptr()), ws_bytes))
    _call(F, ops, "glt_adamw_graft_step_noalloc", b, 2, 1.0, ())
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)
    for sa, sb in zip(a[0], b[0]):
        for x, y in ((sa.gate, sb.gate), (sa.up, sb.up), (sa.down, sb.down), (sa.packed, sb.packed)):
            assert torch.equal(bits(x), bits(y))
    for xs, ys in ((a[2], b[2]), (a[3], b[3])):
        for x, y in zip(xs, ys):
            assert torch.equal(bits(x), bits(y))


def test_noalloc_graft_step_in_a_hip_graph(dev):
    """The allocation-free step captured in a HIP graph (its scratch address
    baked into the captured launches) and replayed twice, with eager work
    and synchronizations between the replays: each replay equals the eager
    call on a copy of the same state bit for bit."""
    import torch
    from glt_amd import _ffi as F
    from glt_amd import ops
    shapes = [(128, 256), (64, 96)]
    a = _state(torch, ops, shapes, 90)
    b = _clone(torch, ops, a)
    _call(F, ops, "glt_adamw_graft_step_noalloc", a, 5, 0.5, ())     # first call: the scratch lookup
    _call(F, ops, "glt_adamw_graft_step_noalloc", b, 5, 0.5, ())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _call(F, ops, "glt_adamw_graft_step_noalloc", a, 5, 0.5, ())
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)
    for rep in range(2):
        print("noalloc graph replay", rep, flush=True)
        graph.replay()
        torch.cuda.synchronize()
        _call(F, ops, "glt_adamw_graft_step_noalloc", b, 5, 0.5, ())     # eager, on the copy
        torch.cuda.synchronize()
        for sa, sb in zip(a[0], b[0]):
            for x, y in ((sa.gate, sb.gate), (sa.up, sb.up), (sa.down, sb.down), (sa.packed, sb.packed)):
                assert torch.equal(bits(x), bits(y)), rep
        for xs, ys in ((a[2], b[2]), (a[3], b[3])):
            for x, y in zip(xs, ys):
                assert torch.equal(bits(x), bits(y)), rep
    del graph


_FRESH = r"""
import ctypes, sys, torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
from glt_amd import _ffi as F
from glt_amd import ops
import test_zz_no_alloc as T
st = T._state(torch, ops, [(128, 256), (64, 96)], 70)
# the workspace form launches kernels of the same source file, which loads
# its code object (and with it the scratch array) onto the device
ws = torch.empty(F.load().glt_adamw_workspace_size(0), dtype=torch.uint8, device="cuda")
T._call(F, ops, "glt_adamw_graft_step", T._clone(torch, ops, st), 1, 1.0, (ctypes.c_void_p(ws.data_ptr()), ws.numel()))
torch.cuda.synchronize()
free0 = torch.cuda.mem_get_info()[0]
T._call(F, ops, "glt_adamw_graft_step_noalloc", st, 1, 1.0, ())
torch.cuda.synchronize()
free1 = torch.cuda.mem_get_info()[0]
print("free", free0, free1, flush=True)
sys.exit(0 if free0 == free1 else 3)
"""


def test_noalloc_first_call_allocates_nothing(dev):
    """In a fresh process, after the workspace form has run (loading the code
    object that holds the scratch array: 2 MiB of device memory, taken at the
    first launch from that source file whichever entry point makes it), the
    first allocation-free call (which looks up the scratch address) leaves
    the device's free memory unchanged."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FRESH, root], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout
