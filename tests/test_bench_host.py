"""Host-side pieces of bench.py that need no GPU: the one-GPU guard and the FLOP / byte bookkeeping behind the
node-kernel table."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from mace_onegpu import codegen  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "exactly one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


def _tables():
    from mace_onegpu import model as mm
    return mm.Tables(mm.MaceSpec())


def test_symmetric_contraction_flops_closed_forms():
    """Dense-coefficient count 2 (nu + 1) per non-zero and channel.  Layer 2 (out 0e, inputs 0e+1o+2e+3o): nu = 1 is
    w x_0 (1 non-zero); each nu = 2 path (l, l) -> 0 has the 2l + 1 non-zeros of delta_{ab} / sqrt(2l + 1).  A
    single-path table checks the nu = 3 count against a brute-force count of the coupled tensor."""
    from mace_onegpu import o3
    t = _tables()
    sc2 = t.sc2[0]
    nu12 = {1: 1, 2: sum(2 * l1 + 1 for (_, l1, l2) in sc2[2] if l1 == l2)}
    assert all(p[1] == p[2] for p in sc2[2])                    # only (l, l) pairs couple to 0e
    nu3 = codegen.symc_model_flops({0: {3: sc2[3]}}, [0], C=1)
    assert codegen.symc_model_flops(t.sc2, [0], C=1) == 2 * 2 * nu12[1] + 2 * 3 * nu12[2] + nu3
    # (1 1 -> 0) x 1 -> 1: U[M, a, b, c] = delta_ab delta_cM / sqrt(3): 3 x 3 = 9 non-zeros
    assert codegen.symc_model_flops({1: {3: [("3", 1, 1, 0, 1)]}}, [1], C=1) == 2 * 4 * 9
    # brute force over every index for one generic path
    import itertools
    l1, l2, J, l3, L = 1, 2, 2, 1, 1
    A, B = o3.coupling(l1, l2, J), o3.coupling(J, l3, L)
    nnz = 0
    for M, a, b, c in itertools.product(range(2 * L + 1), range(2 * l1 + 1), range(2 * l2 + 1), range(2 * l3 + 1)):
        v = sum(A[a, b, j] * B[j, c, M] for j in range(2 * J + 1))
        nnz += abs(v) > 1e-12
    assert nnz > 0 and codegen.symc_model_flops({L: {3: [("3", l1, l2, J, l3)]}}, [L], C=1) == 2 * 4 * nnz


def test_published_S1_S2():
    """The dense-coefficient convention (scripts/flop_budget.py) stays published beside the executed counts."""
    assert bench.symc_dense_flops(_tables()) == (915712, 129536)


def test_written_flops_counter():
    """fmaf = 2, other binary * and + = 1, += adds 1, 1.0f * is folded; loads, stores and addressing are not
    counted."""
    body = """k(int n, const float* x) {
  const int node = blockIdx.x * 2 + (threadIdx.x >> 7);
  const float x0 = xp[0];
  const float z0 = 0.5f * x0 * x1 + -0.25f * x2 * x3;
  o0 = fmaf(w0, z0, o0);
  o0 += 1.0f * z0 * x4;
  gx1 = fmaf(0.7f * q0, x1, gx1);
  op[0] = o0;
}"""
    assert codegen.written_flops(body) == (2 + 1 + 2) + 2 + (1 + 1) + (2 + 1)


def test_executed_symc_flops_below_the_dense_count():
    """The generated kernels evaluate the contractions factorised: fewer operations than the dense convention,
    and the backward (input gradient plus the density term) more than the forward."""
    sf = bench.symc_flops_per_row()
    S1d, S2d = bench.symc_dense_flops(_tables())
    assert 0 < sf[(1, "fwd")] < S1d and 0 < sf[(2, "fwd")] < S2d
    assert sf[(1, "bwd")] > sf[(1, "fwd")] and sf[(2, "bwd")] > sf[(2, "fwd")]
    assert sf[(1, "fwd")] % 128 == 0


def test_node_algorithmic_linear_and_symc():
    sf = {(1, "fwd"): 10, (1, "bwd"): 30, (2, "fwd"): 5, (2, "bwd"): 12}
    rows, k_sum, n_in, n_comp, acc, n_w = 1000, 16, 16, 16, 1, 4
    B, F = bench.node_algorithmic("linear", (rows, k_sum, n_in, n_comp, acc, n_w), sf)
    assert F == 2 * 128 * 128 * rows * k_sum
    assert B == 4 * 128 * rows * (16 + 32) + 4 * 128 * 128 * 4
    B, F = bench.node_algorithmic("symc2_bwd", (rows,), sf)
    assert F == rows * 12 and B == 4 * 128 * rows * (16 + 1 + 16) + 12 * rows
    B, F = bench.node_algorithmic("symc1_fwd", (rows,), sf)
    assert F == rows * 10 and B == 4 * 128 * rows * (16 + 4) + 4 * rows


def test_build_counts_symc_ops_from_assembly():
    """The build's assembly count of the straight-line contraction kernels: no packed-FP32 instructions (the build
    disables them) and somewhat fewer operations than written in the source (the compiler folds multiplications by
    constants equal to 1 in fp32 and reassociates)."""
    import pytest
    ops = os.path.join(ROOT, "mace-million_amd", "lib", "kernel_ops.json")
    if not os.path.exists(ops):
        pytest.skip("library not built")
    gen = os.path.join(ROOT, "mace-million_amd", "csrc", "gen")
    for layer in (1, 2):
        asm = codegen.symc_executed_flops(gen, layer, ops_json=ops)
        src = codegen.symc_executed_flops(gen, layer)
        for d in ("fwd", "bwd"):
            assert 0.6 * src[d] <= asm[d] <= src[d], (layer, d, asm[d], src[d])
    assert all(v["packed"] == 0 for v in json.load(open(ops)).values())
