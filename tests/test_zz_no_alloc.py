"""weft_ggml_mul_mat_id_noalloc against weft_ggml_mul_mat_id (GPU).

The no-allocation entry point runs the same kernels as the work-buffer one,
on the library's per-device scratch instead of the caller's buffer, so dst
must agree bit for bit on the same inputs.  Two calls in a row, the second
smaller, on shapes that take the grouped MFMA path (Q4_K, MXFP4: many pairs
per expert) and the pair GEMV (few pairs); a call whose work size exceeds
the scratch is refused with nothing written."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as o
from weft_amd import ggml as G

pytestmark = pytest.mark.gpu

NAN = 0x7FC00001
TYPE = {"q4_k": G.Q4_K, "mxfp4": G.MXFP4, "q4_0": G.Q4_0}


def case(hip, fmt, k, n, n_as, n_ids, n_tok, seed):
    rb = o.record_bytes(fmt, k)
    w = np.stack([o.quantize(fmt, o.seeded_normal(seed + e, (n, k), 0.02)) for e in range(n_as)])
    x = o.seeded_normal(seed + 50, (n_tok, 1, k))
    ids = np.random.default_rng(seed).integers(0, n_as, size=(n_tok, n_ids)).astype(np.int32)
    wd, xd, idd = hip.to_dev(w), hip.to_dev(x), hip.to_dev(ids)
    s0 = G.tensor(TYPE[fmt], (k, n, n_as), wd.ptr, [G.type_size(TYPE[fmt]), rb, rb * n, rb * n * n_as])
    s1 = G.tensor(G.F32, (k, 1, n_tok), xd.ptr)
    it = G.tensor(G.I32, (n_ids, n_tok), idd.ptr)
    return (wd, xd, idd), s0, s1, it


def run_both(hip, fmt, k, n, n_as, n_ids, n_tok, seed):
    keep, s0, s1, it = case(hip, fmt, k, n, n_as, n_ids, n_tok, seed)
    outs = []
    for noalloc in (False, True):
        yd = hip.empty(4 * n * n_ids * n_tok)
        yd.t[:yd.nbytes].view(hip.torch.int32).fill_(NAN)
        d = G.tensor(G.F32, (n, n_ids, n_tok), yd.ptr)
        print(f"mul_mat_id {fmt} k={k} n={n} n_as={n_as} n_ids={n_ids} n_tok={n_tok} noalloc={noalloc}",
              flush=True)
        if noalloc:
            G.mul_mat_id_noalloc(s0, s1, it, d)
        else:
            wsize = G.mul_mat_id_work_size(s0, s1, it)
            wdata = hip.empty(wsize, fill=0xA5)
            G.mul_mat_id(s0, s1, it, d, wdata.ptr, wsize)
        hip.torch.cuda.synchronize()
        assert hip.last_error() == 0
        outs.append(yd.numpy(np.uint32).copy())
    return outs


@pytest.mark.parametrize("fmt", ["q4_k", "mxfp4", "q4_0"])
def test_noalloc_matches_work_buffer_twice(hip, fmt):
    # first call: 96 tokens x 2 slots over 6 experts (the grouped GEMM);
    # second, smaller: 3 tokens (the pair GEMV), scratch left from the first
    for args in ((1024, 192, 6, 2, 96, 5), (512, 64, 4, 2, 3, 9)):
        ref, got = run_both(hip, fmt, *args)
        assert (ref != NAN).all()
        np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("fmt", ["q4_k", "mxfp4", "q4_0"])
def test_noalloc_long_rows(hip, fmt):
    # four pairs of K = 2^18 rows, past the pair GEMV's LDS: the grouped GEMM
    # takes them whatever the pair count, its grouping in the scratch
    ref, got = run_both(hip, fmt, 1 << 18, 8, 3, 2, 2, 13)
    assert (ref != NAN).all()
    np.testing.assert_array_equal(got, ref)


def test_noalloc_refuses_work_beyond_the_scratch(hip):
    # Q8_K src1 of 32768 tokens x 4096: 37 MB of work buffer > 32 MiB
    k, n, n_tok = 4096, 16, 32768
    s0 = G.tensor(G.Q4_K, (k, n, 2), 0, [G.type_size(G.Q4_K), o.record_bytes("q4_k", k),
                                         o.record_bytes("q4_k", k) * n, o.record_bytes("q4_k", k) * n * 2])
    s1 = G.tensor(G.F32, (k, 1, n_tok), 0)
    it = G.tensor(G.I32, (1, n_tok), 0)
    assert G.mul_mat_id_work_size(s0, s1, it) > G.NOALLOC_SCRATCH_BYTES
    yd = hip.empty(4 * n * n_tok, fill=0x5A)
    d = G.tensor(G.F32, (n, 1, n_tok), yd.ptr)
    with pytest.raises(Exception, match="weft_ggml_mul_mat_id_noalloc"):
        G.mul_mat_id_noalloc(s0, s1, it, d)
    hip.torch.cuda.synchronize()
    assert hip.last_error() == 0
    assert (yd.numpy(np.uint8) == 0x5A).all()
