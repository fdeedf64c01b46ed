"""GPU: the allocation-free sampling entry (pulsar_sample_rows_static) against the entry it
varies (pulsar_sample_rows with a caller workspace), through the C ABI.

Two calls in a row, the second with fewer rows and sequences than the first (the static
scratch keeps the first call's contents), in bf16 and fp32 rounding, sampled and greedy:
penalised argmax and both draws identical to the workspace entry's, element for element.
Requests beyond the scratch's 4096 sequences are refused with a message.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(n_rows, n_seq, V, seed):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(n_rows, V, generator=g) * 3.0).cuda()
    bits = torch.randint(0, 2 ** 31 - 1, (n_seq, V // 32), generator=g, dtype=torch.int32)
    bits &= torch.randint(0, 2 ** 31 - 1, (n_seq, V // 32), generator=g, dtype=torch.int32)
    row_seq = torch.randint(0, n_seq, (n_rows,), generator=g, dtype=torch.int32)
    row_extra = torch.randint(-1, V, (n_rows,), generator=g, dtype=torch.int32)
    ctr = torch.randint(0, 1000, (n_seq,), generator=g, dtype=torch.int32)
    return [t.cuda() for t in (logits, bits, row_seq, row_extra, ctr)]


def _call(lib, static, ins, V, dtype, seed, T, top_p, rp, greedy):
    from pulsar_cuda import _lib

    logits, bits, row_seq, row_extra, ctr = ins
    n_rows, n_seq = logits.shape[0], bits.shape[0]
    am = torch.full((n_rows,), -7, dtype=torch.int32, device="cuda")
    dr = torch.full((n_rows, 2), -7, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    args = [logits.data_ptr(), n_rows, V, dtype, bits.data_ptr(), row_seq.data_ptr(),
            row_extra.data_ptr(), ctr.data_ptr(), n_seq, seed, T, top_p, rp, int(greedy),
            am.data_ptr(), dr.data_ptr()]
    if static:
        _lib.check(lib.pulsar_sample_rows_static(*args, stream))
    else:
        ws = torch.empty(int(lib.pulsar_sample_workspace_bytes(n_seq)), dtype=torch.uint8,
                         device="cuda")
        _lib.check(lib.pulsar_sample_rows(*args, ws.data_ptr(), stream))
        torch.cuda.synchronize()
        del ws
    torch.cuda.synchronize()
    return am.cpu().numpy(), dr.cpu().numpy()


@pytest.mark.parametrize("dtype_name", ["bf16", "fp32"])
def test_static_entry_equals_workspace_entry_on_two_calls(dtype_name):
    from pulsar_cuda import _lib

    lib = _lib.load()
    dtype = _lib.PULSAR_BF16 if dtype_name == "bf16" else _lib.PULSAR_F32
    V = 32768
    for greedy in (False, True):
        for i, (n_rows, n_seq) in enumerate(((192, 96), (7, 3))):
            ins = _inputs(n_rows, n_seq, V, seed=100 * i + int(greedy))
            kw = dict(V=V, dtype=dtype, seed=12345 + i, T=0.8, top_p=0.95, rp=1.15, greedy=greedy)
            want = _call(lib, False, ins, **kw)
            got = _call(lib, True, ins, **kw)
            assert (want[0] >= 0).all() and (want[1] >= 0).all()
            np.testing.assert_array_equal(got[0], want[0])
            np.testing.assert_array_equal(got[1], want[1])
            if not greedy:
                assert (want[1][:, 0] != want[0]).any() or n_rows < 16


def test_static_entry_refuses_more_sequences_than_its_scratch():
    from pulsar_cuda import _lib

    lib = _lib.load()
    V = 4096
    ins = _inputs(4, 4097, V, seed=1)
    with pytest.raises(RuntimeError, match="4096"):
        _call(lib, True, ins, V=V, dtype=_lib.PULSAR_F32, seed=1, T=0.8, top_p=0.9, rp=1.1,
              greedy=False)
