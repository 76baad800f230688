"""Maximum sizes: the address arithmetic at the limits of each path.

The unmasked staged kernels address A, B and C with 64-bit offsets, so a
matrix may exceed 2^31 elements.  Those that stage through buffer loads take a
32-bit byte offset from each slab's base, which covers BM rows of A and BK rows
of B while BM * K + BK and BK * N + BN stay below 2^29 elements; past that the
launch runs the same loop with flat 64-bit loads.  The masked twins use 32-bit
offsets and the host rejects problems whose tiles could reach 2^31 elements
((M + 256) * K or (K + 64) * (N + 256), runtime select_launches).

With entries in {-1, 0, 1} and K < 2^24 every partial sum is an integer that
float32 holds exactly, so the product is exact in any summation order and
must equal PyTorch's float32 GEMM of the same matrices bit for bit; the
epilogue (integer bias, IEEE relu) keeps it exact.
"""

import numpy as np
import pytest

from tensorforge_amd import _lib
from tensorforge_amd import tforge_cpu as tc

STAGED = "block-tile={},{} thread-tile={},{} tile-k={} promote=1 vectorize=1"


def _exact_case(m, n, k, options):
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(11)
    a = torch.randint(-1, 2, (m, k), device=dev, generator=g, dtype=torch.int8).float()
    b = torch.randint(-1, 2, (k, n), device=dev, generator=g, dtype=torch.int8).float()
    bias = torch.randint(-64, 65, (n,), device=dev, generator=g, dtype=torch.int32).float()
    kern = _lib.Kernel(tc.gen_mlir("mbr", m, n, k), options, "t.mlir")
    out = torch.full((m, n), float("nan"), device=dev)
    kern.launch([a.data_ptr(), b.data_ptr(), bias.data_ptr(), out.data_ptr()],
                torch.cuda.current_stream().cuda_stream)
    # The reference product in column chunks: PyTorch's own GEMM returned
    # wrong rows for a 128 x 2^25 output on this stack.
    want = torch.empty_like(out)
    for j in range(0, n, 1 << 20):
        want[:, j:j + (1 << 20)] = torch.mm(a, b[:, j:j + (1 << 20)].contiguous())
    want.add_(bias).relu_()
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    assert torch.equal(out.view(torch.int32), want.view(torch.int32))
    # the exact result really is the integer product: spot-check corners in float64
    for i, j in ((3, 5), (m - 1, n - 1), (m - 2, n // 2 + 1)):
        assert float(out[i, j]) == max(0.0, float((a[i].double() * b[:, j].double()).sum()) + float(bias[j]))


@pytest.mark.gpu
def test_unmasked_kernel_past_2_31_elements():
    """A is 512 x 2^23 = 2^32 elements (16 GiB): 64-bit offsets in A; split-K
    over 64 K ranges fills the GPU."""
    _exact_case(512, 128, 1 << 23, STAGED.format(128, 128, 8, 4, 32) + " split-k=64")


@pytest.mark.gpu
def test_masked_kernel_at_its_2_31_limit():
    """(M + 256) * K is 65,648 elements below 2^31, K is not a multiple of the
    K tile (guarded tail slab), M and N are ragged."""
    m, n, k = 257, 65, 4186000
    assert (m + 256) * k < 1 << 31 and (m + 256) * k > (1 << 31) - 70000
    _exact_case(m, n, k, STAGED.format(64, 64, 4, 4, 32) + " mask-edges=1 split-k=16")


def test_masked_kernel_past_its_limit_is_refused():
    """One more K row per 513 and the host refuses the masked twin with the
    documented message (no GPU needed)."""
    m, n, k = 257, 65, 4186200
    assert (m + 256) * k >= 1 << 31
    with pytest.raises(RuntimeError, match="mask-edges supports matrices below 2\\^31"):
        _lib.Kernel(tc.gen_mlir("mbr", m, n, k), STAGED.format(64, 64, 4, 4, 32) + " mask-edges=1", "t.mlir")


# The spread-staging 128 x 128 kernel (thread-tile 8,8, tile-k 16) on both
# sides of its buffer-load limit: BM * K + BK (A) or BK * N + BN (B) just below
# 2^29 elements runs buffer loads whose byte offsets reach 2^31 - 64 KiB or
# more; one K tile (or one N tile) more runs the flat-load loop.
SPREAD_88 = STAGED.format(128, 128, 8, 8, 16)


@pytest.mark.gpu
@pytest.mark.parametrize("k", [4194288, 4194320])
def test_buffer_load_limit_in_a(k):
    assert (128 * k + 16 < 1 << 29) == (k == 4194288)
    _exact_case(128, 128, k, SPREAD_88 + " split-k=8")


@pytest.mark.gpu
@pytest.mark.parametrize("n", [33554304, 33554432])
def test_buffer_load_limit_in_b(n):
    """B is 96 x ~2^25 (12 GiB), C 128 x ~2^25 (16 GiB); six K slabs, so the
    slab loop's own loads (slabs 3 to 5) take the path under test."""
    assert (16 * n + 128 < 1 << 29) == (n == 33554304)
    _exact_case(128, n, 96, SPREAD_88)
