"""The sparse decode variant that allocates nothing (xt_sparse_decode_nvfp4_static, the library's fixed per-GPU array as
its workspace), through the C ABI, against xt_sparse_decode_nvfp4 with a caller workspace: outputs and LSE bit for
bit on two calls in a row, the second smaller than the first, and a clear error beyond the array's size."""
import numpy as np
import pytest
import torch

from tests._pools import Pool
from xtier_amd import _lib, ops, workloads

pytestmark = pytest.mark.gpu


def _case(seed, batch, heads=4, qh=32, ctx=3008, topk=700, page=64):
    gen = workloads.generator('cpu', seed)
    k = workloads.kv_tensor(batch * ctx, heads, 128, gen, 'cpu')
    v = workloads.kv_tensor(batch * ctx, heads, 128, gen, 'cpu')
    pt = workloads.page_table(batch, ctx, page, gen, 'cpu').cuda()
    idx = workloads.index_lists(batch, ctx, topk, gen, 'cpu')
    idx[0, ::11] = -1
    q = (torch.randn(batch, qh, 128, generator=gen) * 2).to(torch.bfloat16).cuda()
    seq = torch.full((batch,), ctx, dtype=torch.int32, device='cuda')
    return Pool(k, v), pt, idx.cuda(), q, seq


def test_static_workspace_equals_caller_workspace_on_consecutive_calls():
    for seed, batch, splits in ((1, 12, 5), (2, 3, 2)):     # the second call is smaller than the first
        pool, pt, idx, q, seq = _case(seed, batch)
        outs, lses = [], []
        for ws in ('static', ops.new_workspace('cuda', batch, 32, 128, splits)):
            out = torch.empty(batch, 32, 128, dtype=torch.bfloat16, device='cuda')
            lse = torch.empty(batch, 32, dtype=torch.float32, device='cuda')
            ops.sparse_decode(q, pool.raw, pt, idx, seq, 0.0884, page_size=64, out=out, lse=lse, splits=splits,
                              ws=ws)
            outs.append(out)
            lses.append(lse)
        torch.cuda.synchronize()
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), (batch, splits)
        assert torch.equal(lses[0].view(torch.int32), lses[1].view(torch.int32)), (batch, splits)


def test_static_workspace_rejects_shapes_beyond_its_size():
    pool, pt, idx, q, seq = _case(3, 2)
    rows, splits = 512, 4           # 64 KB + 512 x 4 x 32 x 132 x 4 bytes: beyond 8 MiB
    assert ops.decode_workspace_bytes(rows, 32, 128, splits) > 8 << 20
    k, v, ksf, vsf, gk, gv = pool.raw
    st = _lib.lib().xt_sparse_decode_nvfp4_static(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), ksf.data_ptr(), vsf.data_ptr(),
        gk.data_ptr(), gv.data_ptr(), k.shape[0], 0, 0, 0, 0, 4, 32, 128, pt.data_ptr(), pt.stride(0), 64, None,
        idx.data_ptr(), idx.stride(0), idx.shape[1], None, seq.data_ptr(), None, 0.0884, q.data_ptr(), 0, 0,
        _lib.XT_DTYPE_BF16, None, rows, splits, torch.cuda.current_stream().cuda_stream)
    assert st == _lib.XT_EWORKSPACE and b'8388608' in _lib.lib().xt_last_error()
    np.testing.assert_equal(st, _lib.XT_EWORKSPACE)
