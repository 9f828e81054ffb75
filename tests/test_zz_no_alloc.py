"""gemm_noalloc (include/gemm.h): gemm() that allocates nothing, its split-K
partials in a fixed 64 MiB device array of the library, for callers that
cannot call hipMalloc (graph capture, serving loops). Through the C-ABI:

  * two calls in a row, the second with a smaller problem (the array keeps
    the first call's partials): each equals gemm() on the null stream bit for
    bit (both split K the same way: these partials fit the array), on the
    null stream and on a non-null stream, where gemm() itself does not split
    (so the bits differ from gemm() there: the variant did split);
  * each is within the bf16x3 summation bound of the split's exact value
    (gemm() runs on bf16x3 products);
  * the device's free memory is the same before and after the calls.
"""
import numpy as np
import pytest

import bmb
import oracle as O
from gpu_util import bf16x3_err

pytestmark = pytest.mark.gpu

# (M, N, K, transA, transB): few output tiles against K, so the planner
# splits K; the second problem is smaller than the first.
CASES = [(768, 768, 8192, True, False), (257, 129, 3000, False, False)]


def _bits(t):
    return t.cpu().numpy().view(np.uint32).copy()


def test_noalloc_matches_gemm(gpu):
    import torch
    f32 = dict(device="cuda", dtype=torch.float32)
    side = torch.cuda.Stream()
    data = []
    for i, (M, N, K, ta, tb) in enumerate(CASES):
        A = O.fill_xorshift(M * K, 0x4242 + i)
        B = O.fill_xorshift(K * N, 0x5353 + i)
        C0 = O.fill_xorshift(M * N, 0x6464 + i)
        d = {"A": torch.from_numpy(A).to(**f32), "B": torch.from_numpy(B).to(**f32),
             "C0": torch.from_numpy(C0).to(**f32), "C": torch.empty(M * N, **f32)}
        # references from gemm(): null stream (splits K in leased scratch) and
        # a non-null stream (no split)
        d["C"].copy_(d["C0"])
        bmb.gemm(ta, tb, M, N, K, 0.75, d["A"].data_ptr(), d["B"].data_ptr(), 1.25,
                 d["C"].data_ptr())
        torch.cuda.synchronize()
        d["ref"] = _bits(d["C"])
        d["C"].copy_(d["C0"])
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            bmb.gemm(ta, tb, M, N, K, 0.75, d["A"].data_ptr(), d["B"].data_ptr(), 1.25,
                     d["C"].data_ptr(), side.cuda_stream)
        side.synchronize()
        d["nosplit"] = _bits(d["C"])
        bmb.check("gemm references")
        d["host"] = (A, B, C0)
        data.append(d)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]

    for stream in (None, side):
        for (M, N, K, ta, tb), d in zip(CASES, data):
            print("gemm_noalloc %s M=%d N=%d K=%d on the %s stream"
                  % ("TN" if ta else "NN", M, N, K, "null" if stream is None else "side"),
                  flush=True)
            d["C"].copy_(d["C0"])
            torch.cuda.synchronize()
            rc = bmb.call("gemm_noalloc", ta, tb, M, N, K, 0.75, d["A"].data_ptr(),
                          d["B"].data_ptr(), 1.25, d["C"].data_ptr(),
                          None if stream is None else stream.cuda_stream)
            assert rc == 0
            torch.cuda.synchronize()
            bmb.check("gemm_noalloc")
            got = _bits(d["C"])
            assert np.array_equal(got, d["ref"])
            assert not np.array_equal(got, d["nosplit"])
            A, B, C0 = d["host"]
            err, bound = bf16x3_err(got.view(np.float32), ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
            assert err < bound, (err, bound)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    print("free memory before %.1f MiB, after %.1f MiB" % (free0 / 2**20, free1 / 2**20))
    assert free1 == free0
