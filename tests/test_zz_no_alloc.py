"""The allocation-free reorder, kv_reorder_noalloc_dev, through the C ABI:
bit for bit kv_reorder_dev with caller temporaries (and numpy's gather),
on two calls in a row, the second smaller (the library's one device array
keeps the first call's contents), and a shape whose temporaries exceed the
array refused."""

import numpy as np
import pytest

from go_whistle_amd import cq, synth
from go_whistle_amd._lib import CQPanic, check, lib

pytestmark = pytest.mark.gpu


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _p(t):
    from ctypes import c_void_p

    return c_void_p(t.data_ptr())


def _case(g, B, cap, cols, width):
    q = g.integers(-128, 128, size=(B, cap, cols), dtype=np.int8)
    s = g.random((B, cap, cols // width)).astype(np.float32)
    parent = g.integers(0, B, size=B).astype(np.int32)
    ln = g.integers(0, cap + 2, size=B).astype(np.int32)  # past cap: clamped
    ln[0] = cap
    return q, s, parent, ln


def _both(q, s, parent, ln, cols, width):
    import torch

    B, cap = q.shape[0], q.shape[1]
    qa, sa, qb, sb = _t(q), _t(s), _t(q), _t(s)
    pd, ld = _t(parent), _t(ln)
    tq, ts = torch.empty_like(qa), torch.empty_like(sa)
    st = cq._stream()
    check(lib().kv_reorder_dev(_p(qa), _p(sa), _p(tq), _p(ts), _p(pd), _p(ld), B, cap, cols, width, st))
    check(lib().kv_reorder_noalloc_dev(_p(qb), _p(sb), _p(pd), _p(ld), B, cap, cols, width, st))
    torch.cuda.synchronize()
    return qa.cpu().numpy(), sa.cpu().numpy(), qb.cpu().numpy(), sb.cpu().numpy()


def test_noalloc_reorder_matches_the_allocating_one():
    g = synth.rng(2026)
    for B, cap, cols, width in ((64, 200, 512, 64), (5, 7, 40, 8)):  # the second call smaller, odd widths
        q, s, parent, ln = _case(g, B, cap, cols, width)
        qa, sa, qb, sb = _both(q, s, parent, ln, cols, width)
        assert np.array_equal(qb, qa) and np.array_equal(sb.view(np.uint32), sa.view(np.uint32))
        wq, ws = q.copy(), s.copy()
        for b in range(B):
            n = min(int(ln[b]), cap)
            wq[b, :n], ws[b, :n] = q[parent[b], :n], s[parent[b], :n]
        assert np.array_equal(qb, wq) and np.array_equal(sb.view(np.uint32), ws.view(np.uint32))


def test_noalloc_reorder_refuses_more_than_its_array():
    import torch

    z = torch.zeros(16, dtype=torch.int32, device="cuda")
    # 256 streams x 128 rows x 512 codes = 16 MiB of codes alone, plus scales
    with pytest.raises(CQPanic) as e:
        check(lib().kv_reorder_noalloc_dev(_p(z), _p(z), _p(z), _p(z), 256, 128, 512, 64, cq._stream()))
    assert "16777216" in str(e.value)
