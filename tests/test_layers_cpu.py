"""SplitKLinear host logic on the CPU: the slice choice and the F.linear
fallback for inputs split-K cannot view (CPU tensors, strided rows)."""
import torch

from tinyvllm.layers import SplitKLinear


def test_splits_for_table():
    cases = {  # (in, out): slices at rows 1, 128, 129, 512, 513
        (3072, 1024): (8, 8, 2, 2, 1),
        (4096, 4096): (4, 4, 4, 4, 1),
        (12288, 4096): (4, 4, 8, 8, 1),
        (25600, 5120): (4, 4, 8, 8, 1),
        (100, 4096): (1, 1, 1, 1, 1),  # reduction not divisible into slices
    }
    for (k, n), expect in cases.items():
        lin = SplitKLinear(k, n, device="meta")
        assert tuple(lin.splits_for(r) for r in (1, 128, 129, 512, 513)) == expect, (k, n)


def test_cpu_and_strided_inputs_take_linear():
    torch.manual_seed(0)
    lin = SplitKLinear(256, 64)
    x = torch.randn(8, 512)[:, ::2]
    y = lin(x)
    assert isinstance(y, torch.Tensor)
    torch.testing.assert_close(y, torch.nn.functional.linear(x, lin.weight))
    y2 = lin(x.contiguous())
    torch.testing.assert_close(y2, torch.nn.functional.linear(x.contiguous(), lin.weight))
