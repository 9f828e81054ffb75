"""gemm_noalloc (include/gemm.h): gemm() that allocates nothing, its split-K
partials in a fixed 64 MiB device array of the library, for callers that
cannot call hipMalloc (graph capture, serving loops). Through the C-ABI:

  * two calls in a row, the second with a smaller problem (the array keeps
    the first call's partials): each equals gemm() bit for bit (both split K
    the same way: these partials fit the array), on the null stream and on a
    non-null stream, in both arithmetic modes of gemm_set_math();
  * a problem whose gemm() split needs more than the array (2560 x 2560 x
    16384: five K ranges, 125 MiB of partials) runs on a plan capped to the
    array: different bits from gemm(), within the same bound;
  * each result is within its mode's bound (the bf16x3 summation bound of
    the split's exact value, or the fp32 summation bound of the product);
  * a call captured into a HIP graph on a side stream and replayed three
    times, with eager work between the replays, gives the eager call's bits
    every time;
  * the device's free memory is the same before and after all of it.
"""
import numpy as np
import pytest

import bmb
import oracle as O
from gpu_util import bf16x3_err, fp32_order_bound

pytestmark = pytest.mark.gpu

# (M, N, K, transA, transB): few output tiles against K, so the planner
# splits K; the second problem is smaller than the first.
CASES = [(768, 768, 8192, True, False), (257, 129, 3000, False, False)]
CAPPED = (2560, 2560, 16384, False, False)


def _bits(t):
    return t.cpu().numpy().view(np.uint32).copy()


def _problem(torch, i, M, N, K):
    f32 = dict(device="cuda", dtype=torch.float32)
    A = O.fill_xorshift(M * K, 0x4242 + i)
    B = O.fill_xorshift(K * N, 0x5353 + i)
    C0 = O.fill_xorshift(M * N, 0x6464 + i)
    return {"A": torch.from_numpy(A).to(**f32), "B": torch.from_numpy(B).to(**f32),
            "C0": torch.from_numpy(C0).to(**f32), "C": torch.empty(M * N, **f32),
            "host": (A, B, C0)}


def _noalloc(d, M, N, K, ta, tb, stream):
    return bmb.call("gemm_noalloc", ta, tb, M, N, K, 0.75, d["A"].data_ptr(),
                    d["B"].data_ptr(), 1.25, d["C"].data_ptr(), stream)


def _within_bound(math, got, M, N, K, ta, tb, host, rows=None):
    A, B, C0 = host
    if rows is not None:  # a row sample of op(A) (rows are independent problems)
        A = np.ascontiguousarray((A.reshape(K, M).T if ta else A.reshape(M, K))[rows])
        C0 = C0.reshape(M, N)[rows]
        got = got.reshape(M, N)[rows]
        M, ta = len(rows), False
    if math == bmb.GEMM_MATH_BF16X3:
        err, bound = bf16x3_err(got, ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    else:
        err, bad = O.normwise(got, O.gemm_f64(ta, tb, M, N, K, 0.75, A, B, 1.25, C0))
        err, bound = (err if bad == 0 else float("inf")), fp32_order_bound(K)
    assert err < bound, (err, bound)


@pytest.mark.parametrize("math", [bmb.GEMM_MATH_BF16X3, bmb.GEMM_MATH_FP32],
                         ids=["bf16x3", "fp32"])
def test_noalloc_matches_gemm(gpu, math):
    import torch
    side = torch.cuda.Stream()
    with bmb.gemm_math(math):
        data = []
        for i, (M, N, K, ta, tb) in enumerate(CASES + [CAPPED]):
            d = _problem(torch, i, M, N, K)
            d["C"].copy_(d["C0"])
            bmb.gemm(ta, tb, M, N, K, 0.75, d["A"].data_ptr(), d["B"].data_ptr(), 1.25,
                     d["C"].data_ptr())
            torch.cuda.synchronize()
            bmb.check("gemm reference")
            d["ref"] = _bits(d["C"])
            # gemm() on the side stream gives the same bits (and the stream's
            # first launch, which sets up runtime resources, happens before
            # the free memory is read)
            d["C"].copy_(d["C0"])
            torch.cuda.synchronize()
            bmb.gemm(ta, tb, M, N, K, 0.75, d["A"].data_ptr(), d["B"].data_ptr(), 1.25,
                     d["C"].data_ptr(), side.cuda_stream)
            side.synchronize()
            bmb.check("gemm reference on the side stream")
            assert np.array_equal(_bits(d["C"]), d["ref"])
            data.append(d)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]

        for stream in (None, side):
            for (M, N, K, ta, tb), d in zip(CASES, data):
                print("gemm_noalloc math %d %s M=%d N=%d K=%d on the %s stream"
                      % (math, "TN" if ta else "NN", M, N, K,
                         "null" if stream is None else "side"), flush=True)
                d["C"].copy_(d["C0"])
                torch.cuda.synchronize()
                assert _noalloc(d, M, N, K, ta, tb,
                                None if stream is None else stream.cuda_stream) == 0
                torch.cuda.synchronize()
                bmb.check("gemm_noalloc")
                got = _bits(d["C"])
                assert np.array_equal(got, d["ref"])
                _within_bound(math, got.view(np.float32), M, N, K, ta, tb, d["host"])

        M, N, K, ta, tb = CAPPED
        d = data[-1]
        print("gemm_noalloc math %d capped plan M=%d N=%d K=%d" % (math, M, N, K), flush=True)
        d["C"].copy_(d["C0"])
        torch.cuda.synchronize()
        assert _noalloc(d, M, N, K, ta, tb, side.cuda_stream) == 0
        torch.cuda.synchronize()
        bmb.check("gemm_noalloc capped")
        got = _bits(d["C"])
        if math == bmb.GEMM_MATH_BF16X3:
            assert not np.array_equal(got, d["ref"])  # another split: the plan was capped
        rows = np.unique(np.r_[0, 1, 255, 256, M // 2, M - 1,
                               np.random.default_rng(9).integers(0, M, 6)])
        _within_bound(math, got.view(np.float32), M, N, K, ta, tb, d["host"], rows)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
    print("free memory before %.1f MiB, after %.1f MiB" % (free0 / 2**20, free1 / 2**20))
    assert free1 == free0


def test_noalloc_in_a_captured_graph(gpu):
    """gemm_noalloc captured on a side stream (torch.cuda.graph) and replayed
    three times; C is reset eagerly and other eager GEMMs run between the
    replays. Every replay gives the eager call's bits, and the replays leave
    the free memory unchanged (measured after the first one: instantiating
    the graph may itself hold device memory)."""
    import torch
    M, N, K, ta, tb = CASES[0]
    d = _problem(torch, 0, M, N, K)
    other = _problem(torch, 1, *CASES[1][:3])
    side = torch.cuda.Stream()
    # eager call first: resolves the array's address and the planner's
    # per-device tables outside the capture
    d["C"].copy_(d["C0"])
    torch.cuda.synchronize()
    assert _noalloc(d, M, N, K, ta, tb, side.cuda_stream) == 0
    side.synchronize()
    bmb.check("gemm_noalloc eager")
    ref = _bits(d["C"])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("capturing gemm_noalloc TN %dx%dx%d" % (M, N, K), flush=True)
    with torch.cuda.graph(g, stream=side):
        rc = _noalloc(d, M, N, K, ta, tb, side.cuda_stream)
    assert rc == 0
    bmb.check("gemm_noalloc capture")
    for r in range(3):
        d["C"].copy_(d["C0"])
        torch.cuda.synchronize()
        print("replay %d" % r, flush=True)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(d["C"]), ref)
        # eager work between replays (it uses the same array)
        Mo, No, Ko, tao, tbo = CASES[1]
        other["C"].copy_(other["C0"])
        assert _noalloc(other, Mo, No, Ko, tao, tbo, None) == 0
        torch.cuda.synchronize()
        bmb.check("gemm_noalloc between replays")
        if r == 0:
            free0 = torch.cuda.mem_get_info()[0]
    free1 = torch.cuda.mem_get_info()[0]
    del g
    print("free memory after replay 0 %.1f MiB, after replay 2 %.1f MiB"
          % (free0 / 2**20, free1 / 2**20))
    assert free1 == free0
