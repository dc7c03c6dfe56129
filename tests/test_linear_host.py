"""Host side of the MFMA linear (no GPU): the three-way bf16 split of the weights and the B-operand order of the
weight blocks that mm_linear stages in LDS."""
import torch

from mace_onegpu.fast_layers import mfma_block, split3_bf16


def test_split_reconstructs_fp32_to_2_pow_minus_27():
    g = torch.Generator().manual_seed(0)
    W = torch.randn(128, 128, generator=g) * torch.logspace(-6, 6, 128)[:, None]
    w0, w1, w2 = split3_bf16(W)
    assert w0.dtype == w1.dtype == w2.dtype == torch.bfloat16
    rec = w0.double() + w1.double() + w2.double()
    err = (rec - W.double()).abs()
    assert bool((err <= 2.0 ** -27 * W.double().abs()).all())
    # the pieces shrink by at least 2^-8 each (round to nearest: |W - W0| <= 2^-9 |W|)
    assert bool((w1.double().abs() <= 2.0 ** -8 * W.double().abs()).all())
    assert bool((w2.double().abs() <= 2.0 ** -16 * W.double().abs()).all())
    # values a bf16 holds exactly split into (W, 0, 0)
    e = torch.tensor([1.0, -0.5, 3.0, 2.0 ** -20])
    a, b, c = split3_bf16(e)
    assert torch.equal(a.float(), e) and not b.float().any() and not c.float().any()


def test_block_order_is_the_b_operand_layout():
    """Plane p, lane (i, g), K-step t, tile nt reads 8 consecutive bf16 at uint4 index ((t * 8 + nt) * 4 + g) * 16 + i:
    they must be W_p[32 t + 8 g + u][16 nt + i], u = 0..7."""
    W = torch.arange(128 * 128, dtype=torch.float32).reshape(128, 128) / 7.0
    blk = mfma_block(W)
    assert blk.shape == (3 * 16384,) and blk.dtype == torch.bfloat16
    planes = split3_bf16(W)
    for p in range(3):
        plane = blk[p * 16384:(p + 1) * 16384].view(2048, 8)
        for (t, nt, g, i) in [(0, 0, 0, 0), (3, 7, 3, 15), (1, 2, 3, 4), (2, 5, 0, 9)]:
            got = plane[((t * 8 + nt) * 4 + g) * 16 + i]
            want = planes[p][32 * t + 8 * g:32 * t + 8 * g + 8, 16 * nt + i]
            assert torch.equal(got, want)
    # the order is a permutation: the plane sums are the matrix sums
    for p in range(3):
        assert torch.isclose(blk[p * 16384:(p + 1) * 16384].double().sum(), planes[p].double().sum(), rtol=1e-12)


def test_ace_gb_order_is_the_backward_operand_order():
    """mm_ace1_bwd's lane (m, g) reads 16 contiguous values per species block s, the operands of K-steps k = 0..15:
    position s * 64 + 16 g + k of its gB row must hold feature q = 4 k + g (every feature once per block)."""
    from mace_onegpu.fast_layers import ace_gb_order
    for S_pad in (2, 4):
        order = ace_gb_order(S_pad)
        assert sorted(order.tolist()) == list(range(S_pad * 64))
        row = torch.arange(S_pad * 64)[order]          # what a gB row in operand order holds at each position
        for s in range(S_pad):
            for g in range(4):
                lane = row[s * 64 + 16 * g:s * 64 + 16 * g + 16]
                assert lane.tolist() == [s * 64 + 4 * k + g for k in range(16)]
