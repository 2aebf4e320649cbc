"""The committed golden fixtures: the oracle still reproduces them (CPU), and the kernels match them (GPU)."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from tests.golden import make_golden

HERE = Path(__file__).resolve().parent / 'golden'


def _load(name):
    with np.load(HERE / name) as d:
        return {k: d[k] for k in d.files}


@pytest.mark.parametrize('name,make', [('nvfp4_encode.npz', make_golden.encode_case),
                                       ('decode_small.npz', make_golden.decode_case)])
def test_oracle_reproduces_fixture(name, make):
    want = _load(name)
    got = make()
    assert set(got) == set(want)
    for k in want:
        assert np.array_equal(np.asarray(got[k]), want[k]), k


@pytest.mark.gpu
def test_decode_matches_fixture():
    from xtier_amd import ops
    d = _load('decode_small.npz')
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    raw = (dev(d['k_pay']), dev(d['v_pay']), dev(d['k_sf']), dev(d['v_sf']), dev(d['gk']), dev(d['gv']))
    q = dev(d['q_bf16'].view(np.int16)).view(torch.bfloat16)
    lse = torch.empty(q.shape[:2], dtype=torch.float32, device='cuda')
    out = ops.sparse_decode(q, raw, dev(d['page_table']), dev(d['indices']), dev(d['seq_lens']),
                            float(d['scale'][0]), page_size=64, lse=lse)
    err = np.abs(out.float().cpu().numpy() - d['out'])
    assert err.max() <= 2e-2 and err.mean() <= 2e-3
    assert np.abs(lse.cpu().numpy() - d['lse']).max() < 2e-3
    assert math.isfinite(float(out.float().abs().max()))
