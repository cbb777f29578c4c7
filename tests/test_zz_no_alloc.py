"""``ctmr_conv3d_noalloc`` (the allocation-free variant of ``ctmr_conv3d``) through the C ABI.

Its workspace is the library's own per-GPU scratch array; the output must equal ``ctmr_conv3d``'s
(caller workspace, same kernels) bit for bit, on consecutive calls whose second input is smaller
(the scratch keeps the previous call's contents), on calls alternating between two streams (the
library chains them through a per-device event), and when recorded in a HIP graph (with and
without an eager call first); a convolution whose workspace exceeds the scratch limit must be
refused before anything is launched.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _g(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _case(ctmr, dev, seed, shape, cout, *, mode=0, affine=True, batch_bias=True, residual=True):
    """Inputs of one conv, its output through ctmr_conv3d (ops.conv3d) and the noalloc call's arguments."""
    L, ops = ctmr._lib, ctmr.ops
    rng = np.random.default_rng(seed)
    n, d, h, w, cin = shape
    x = _g(rng.standard_normal(shape).astype(np.float32), dev)
    wt = _g((rng.standard_normal((cout, cin, 3, 3, 3)) / np.sqrt(27 * cin)).astype(np.float32), dev)
    packed = (ctmr.fast_fp32.pack_upsample_weight if mode == L.MODE_NEAREST2X else ctmr.fast_fp32.pack_weight)(
        wt, dtype="fp32")
    bias = _g(rng.standard_normal((n, cout) if batch_bias else (cout,)).astype(np.float32), dev)
    aff = _g(np.stack([1 + 0.2 * rng.standard_normal((n, cin)), 0.3 * rng.standard_normal((n, cin))],
                      axis=-1).astype(np.float32), dev) if affine else None
    desc = ops.make_desc(shape, cout, 3, 1, mode, 0, L.DT_F32, 0)
    od, oh, ow = L.output_dims(desc)
    res = _g(rng.standard_normal((n, od, oh, ow, cout)).astype(np.float32), dev) if residual else None
    ref = ops.conv3d(x, packed, bias, aff, res, cout, 3, 1, mode, affine, L.DT_F32, 0)
    flags = ops._flags(affine, affine, batch_bias, residual)
    desc = ops.make_desc(shape, cout, 3, 1, mode, flags, L.DT_F32, 0)
    return desc, (x, packed, bias, aff, res), ref


def _noalloc(ctmr, desc, inputs, out):
    x, packed, bias, aff, res = inputs
    ptr = lambda t: None if t is None else t.data_ptr()
    return ctmr._lib.lib().ctmr_conv3d_noalloc(ctypes.byref(desc), x.data_ptr(), packed.data_ptr(), ptr(bias),
                                                ptr(aff), ptr(res), out.data_ptr(),
                                                torch.cuda.current_stream().cuda_stream)


def test_noalloc_equals_conv3d_on_consecutive_calls(ctmr, dev):
    L = ctmr._lib
    cases = [
        # deep level: K split, partial planes in the scratch, GN affine + SiLU, batch bias, residual
        ("split", (2, 8, 8, 4, 512), 512, {}),
        # smaller, nearest-2x parity GEMM over a padded packed copy in the scratch
        ("nearest", (1, 6, 8, 10, 64), 48, {"mode": L.MODE_NEAREST2X}),
        # smaller still: cout <= 4 tap-expanded GEMM (packed copy + tap columns in the scratch)
        ("tap_expand", (1, 5, 6, 7, 32), 4, {"batch_bias": False}),
    ]
    for name, shape, cout, kw in cases:
        desc, inputs, ref = _case(ctmr, dev, len(name), shape, cout, **kw)
        need = L.workspace_bytes(desc)
        print(f"noalloc case {name}: {shape}->{cout} kernel {L.conv_kernel(desc)} workspace {need} B", flush=True)
        assert 0 < need <= L.NOALLOC_SCRATCH_BYTES
        out = torch.full_like(ref, float("nan"))
        assert _noalloc(ctmr, desc, inputs, out) == L.OK, L.last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), name
        out2 = torch.full_like(ref, float("nan"))  # the same call again: same bits
        assert _noalloc(ctmr, desc, inputs, out2) == L.OK
        torch.cuda.synchronize()
        assert torch.equal(out2, ref), name


def test_noalloc_refuses_workspace_above_the_limit(ctmr, dev):
    """Config 2b's packed copy (281 MiB) exceeds the 256 MiB scratch: refused before any launch,
    with a message naming both sizes; null pointers are never touched."""
    L = ctmr._lib
    desc = ctmr.ops.make_desc((1, 64, 64, 64, 256), 128, 3, 1, L.MODE_NEAREST2X, 0, L.DT_F32, 0)
    assert L.workspace_bytes(desc) > L.NOALLOC_SCRATCH_BYTES
    rc = L.lib().ctmr_conv3d_noalloc(ctypes.byref(desc), None, None, None, None, None, None, None)
    assert rc == L.E_WORKSPACE
    assert "scratch limit" in L.last_error() and str(L.NOALLOC_SCRATCH_BYTES) in L.last_error()


def test_noalloc_two_streams_alternating(ctmr, dev):
    """Two different convs issued alternately on two streams, with no host synchronisation between
    them: both use the one scratch array (partial planes of a K split; a padded nearest-2x copy), so
    only the library's event chain keeps them apart.  Every output equals ``ctmr_conv3d``'s."""
    L = ctmr._lib
    da, ia, ra = _case(ctmr, dev, 71, (2, 8, 8, 4, 512), 512)
    db, ib, rb = _case(ctmr, dev, 72, (1, 6, 8, 10, 64), 48, mode=L.MODE_NEAREST2X)
    assert L.conv_split(da) > 1 and L.workspace_bytes(db) > 0
    outs_a = [torch.full_like(ra, float("nan")) for _ in range(4)]
    outs_b = [torch.full_like(rb, float("nan")) for _ in range(4)]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for oa, ob in zip(outs_a, outs_b):
        with torch.cuda.stream(s1):
            assert _noalloc(ctmr, da, ia, oa) == L.OK, L.last_error()
        with torch.cuda.stream(s2):
            assert _noalloc(ctmr, db, ib, ob) == L.OK, L.last_error()
    torch.cuda.synchronize()
    for i, (oa, ob) in enumerate(zip(outs_a, outs_b)):
        assert torch.equal(oa, ra), f"stream 1 call {i}"
        assert torch.equal(ob, rb), f"stream 2 call {i}"


def test_noalloc_in_a_graph_after_an_eager_call(ctmr, dev):
    """Recorded in a HIP graph (after an eager call set the device up) and replayed three times with
    other eager work in between: every replay equals ``ctmr_conv3d`` bit for bit."""
    L = ctmr._lib
    desc, inputs, ref = _case(ctmr, dev, 73, (2, 8, 8, 4, 512), 512)
    out = torch.full_like(ref, float("nan"))
    assert _noalloc(ctmr, desc, inputs, out) == L.OK, L.last_error()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert _noalloc(ctmr, desc, inputs, out) == L.OK, L.last_error()
    for i in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        _case(ctmr, dev, 74 + i, (1, 6, 8, 10, 64), 48)  # eager convs between the replays


_FRESH_PROCESS_GRAPH = """
import ctypes, importlib, sys
import numpy as np, torch
sys.path.insert(0, {repo!r})
sys.path.insert(0, {tests!r})
ctmr = importlib.import_module("mlx-generate-ctmr_amd")
import test_zz_no_alloc as t
dev = torch.device("cuda:0")
L = ctmr._lib
desc, inputs, ref = t._case(ctmr, dev, 77, (2, 8, 8, 4, 512), 512)
out = torch.full_like(ref, float("nan"))
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):  # the process's first noalloc call: set-up happens inside the capture
    rc = t._noalloc(ctmr, desc, inputs, out)
assert rc == L.OK, L.last_error()
for i in range(3):
    out.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), i
print("fresh-process graph ok", flush=True)
"""


def test_noalloc_first_call_inside_a_graph_capture(ctmr, dev):
    """In a fresh process, the first ``ctmr_conv3d_noalloc`` call (which looks up the scratch
    address and creates the ordering event) is made under graph capture; replays equal
    ``ctmr_conv3d``."""
    tests = Path(__file__).resolve().parent
    code = _FRESH_PROCESS_GRAPH.format(repo=str(tests.parent), tests=str(tests))
    print("noalloc fresh-process graph capture: starting child", flush=True)
    proc = subprocess.run([sys.executable, "-c", textwrap.dedent(code)], capture_output=True, text=True,
                          timeout=300, env=dict(os.environ))
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-4000:]
    assert "fresh-process graph ok" in proc.stdout
