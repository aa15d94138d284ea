"""GPU: the allocation-free split-K entry point against the allocating one
(same kernels and plan, so the same bits), two calls in a row with the second
smaller, and its refusal of a call beyond the fixed array."""
import numpy as np
import pytest

import prana_amd as P
from tests.test_c3_attention_gpu import c3_case

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_matches_allocating_entry_on_two_calls():
    for n_seq, ctx in ((8, 9000), (1, 3000)):  # the second call is smaller
        cases = [c3_case(ctx - 13 * i, 900 + ctx + i) for i in range(n_seq)]
        pos = [ctx - 13 * i for i in range(n_seq)]
        q = np.stack([c[0] for c in cases])
        kcs = [P.DeviceArray.from_host(c[1]) for c in cases]
        vcs = [P.DeviceArray.from_host(c[2]) for c in cases]
        ref = P.attention_decode_splitk(q, kcs, vcs, pos, 32, 8, 128)
        got = P.attention_decode_splitk_noalloc(q, kcs, vcs, pos, 32, 8, 128)
        assert same_bits(got, ref), (n_seq, ctx)


def test_noalloc_refuses_calls_beyond_the_array():
    # 16 sequences x 64 heads (groups of 8) at 8100 rows need 16*64*64*130
    # floats, above 2^23: refused before any launch
    n, nh, nkv, hd, ctx = 16, 64, 8, 128, 8100
    kc = P.DeviceArray((ctx + 1, nkv * hd), np.uint16)
    vc = P.DeviceArray((ctx + 1, nkv * hd), np.uint16)
    q = np.zeros((n, nh * hd), np.float32)
    with pytest.raises(P.PranaError, match="scratch floats"):
        P.attention_decode_splitk_noalloc(q, [kc] * n, [vc] * n, [ctx] * n, nh, nkv, hd)
