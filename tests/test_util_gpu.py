"""The op's one-launch utilities through the C ABI: ngdn_transpose (the
per-level parameters' layouts) against torch's transpose, and ngdn_cast_bf16
(the gradients' dtype) against torch's round-to-nearest-even cast; both
compared with torch.equal."""

import pytest
import torch

from nested_recurrent_memory_amd.chunk import _cast_grads, _transpose_last2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_transpose_matches_torch(dtype):
    gen = torch.Generator(device="cuda").manual_seed(5)
    shapes = [(2, 16, 128, 128), (2, 16, 64, 128), (3, 70, 33), (1, 1, 5), (2, 0, 4, 8)]
    xs = [torch.randn(*s, generator=gen, device="cuda").to(dtype) for s in shapes]
    outs = _transpose_last2(xs)
    torch.cuda.synchronize()
    for x, y in zip(xs, outs):
        assert y.shape == x.shape[:-2] + (x.shape[-1], x.shape[-2])
        assert torch.equal(y, x.transpose(-1, -2).contiguous())


def test_cast_matches_torch():
    gen = torch.Generator(device="cuda").manual_seed(6)
    xs = [torch.randn(1000, generator=gen, device="cuda") * 3, torch.randn(4, 257, generator=gen,
                                                                          device="cuda")]
    # ties and large values: 1 + 2^-8 (half an ulp of bf16 at 1), 3 * 2^120
    xs.append(torch.tensor([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 3.0 * 2 ** 120, 0.0],
                           device="cuda"))
    outs = _cast_grads(xs, [torch.bfloat16] * len(xs))
    torch.cuda.synchronize()
    for x, y in zip(xs, outs):
        assert y.dtype == torch.bfloat16 and torch.equal(y, x.to(torch.bfloat16))

