"""HIP graph capture of the product launches: a decode-like sequence of
CSR products (fast and strict, batch 1 and 8, int8 and fp32 weights; the
fast batch-1 products run the merge-path kernel, whose arrival counters the
last arrival clears inside the kernel), a Gemm with bias and Relu through
the allocation-free entry (its op(A)^T staged in the fixed per-device
workspace), and a 2:4 int8 GEMM, captured once on a capture stream and
replayed several times with eager work and synchronisations in between;
every replay must give the eager results bit for bit (the same kernels on
the same data).  None of these launches records a memset or an
allocation; the eager run before the capture builds the weights' derived
copies, so the captured products run on them."""
import sys

import numpy as np
import pytest

from pyflamert_amd import workloads

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


def test_graph_replay_matches_eager(ctx):
    import torch

    ip, ix, q, sc = workloads.csr_int8_lognormal(2048, 3000, 0.3, 0.5, 0.02, seed=1)
    Wi8 = ctx.csr_upload(2048, 3000, ip, ix, q, row_scales=sc)
    ipf, ixf, vf = workloads.csr_uniform(1500, 3000, 0.1, 0.02, seed=2)
    Wf = ctx.csr_upload(1500, 3000, ipf, ixf, vf)
    B = (np.random.default_rng(3).standard_normal((3000, 700)) * 0.05).astype(np.float32)
    B[np.random.default_rng(4).random(B.shape) < 0.8] = 0
    BT = ctx.csr_from_dense(B, transpose=True)
    qw, sw = workloads.sp24_int8_weight(512, 1024, seed=5)
    S = ctx.sp24_pack(qw, sw)
    g = torch.Generator(device="cuda").manual_seed(6)
    x1 = torch.randn((3000, 1), device="cuda", generator=g)
    x8 = torch.randn((3000, 8), device="cuda", generator=g)
    A = torch.randn((64, 3000), device="cuda", generator=g)
    bias = torch.randn(700, device="cuda", generator=g)
    xq = torch.randint(-128, 128, (1024, 256), device="cuda", dtype=torch.int8, generator=g)
    outs = {k: torch.empty(shape, device="cuda", dtype=dt) for k, shape, dt in (
        ("i8_1", (2048, 1), torch.float32), ("i8_8", (2048, 8), torch.float32),
        ("i8_1s", (2048, 1), torch.float32), ("i8_8s", (2048, 8), torch.float32),
        ("f_1", (1500, 1), torch.float32), ("f_8", (1500, 8), torch.float32),
        ("gemm", (64, 700), torch.float32), ("sp24", (512, 256), torch.int32))}

    def run():
        Wi8.spmm_dev(x1.data_ptr(), 1, outs["i8_1"].data_ptr(), mode="fast")
        Wi8.spmm_dev(x8.data_ptr(), 8, outs["i8_8"].data_ptr(), mode="fast")
        Wi8.spmm_dev(x1.data_ptr(), 1, outs["i8_1s"].data_ptr(), mode="strict")
        Wi8.spmm_dev(x8.data_ptr(), 8, outs["i8_8s"].data_ptr(), mode="strict")
        Wf.spmm_dev(x1.data_ptr(), 1, outs["f_1"].data_ptr(), mode="fast")
        Wf.spmm_dev(x8.data_ptr(), 8, outs["f_8"].data_ptr(), mode="strict")
        ctx.gemm_csr_dev(A.data_ptr(), 64, 3000, BT, outs["gemm"].data_ptr(), 1.0, 1.0, bias.data_ptr(), 700,
                         relu=True, noalloc=True)
        S.gemm_i8_dev(xq.data_ptr(), 256, outs["sp24"].data_ptr(), out="i32")

    main = torch.cuda.current_stream().cuda_stream
    ctx.set_stream(main)
    # the allocating entry builds the Gemm weight's sliced-ELL copy, which the
    # allocation-free entry then reads (it builds no copy itself)
    ctx.gemm_csr_dev(A.data_ptr(), 64, 3000, BT, outs["gemm"].data_ptr(), 1.0, 1.0, bias.data_ptr(), 700,
                     relu=True)
    run()
    torch.cuda.synchronize()
    eager = {k: v.clone() for k, v in outs.items()}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        run()
    ctx.set_stream(main)
    for rep in range(4):
        for v in outs.values():
            v.zero_()
        run()  # eager work between replays
        torch.cuda.synchronize()
        for v in outs.values():
            v.fill_(7)
        graph.replay()
        torch.cuda.synchronize()
        say(f"graph replay {rep}")
        for k in outs:
            assert torch.equal(outs[k], eager[k]), (rep, k)
    del graph
    for W in (Wi8, Wf, BT, S):
        W.free()
