"""The allocation-free LoRA gradient entry point (qlora_lora_grad_noalloc): its outputs equal
qlora_lora_grad's (workspace form) bit for bit, on two calls in a row with the second smaller
(the static scratch keeps the first call's partial sums, which must not leak into the second),
and a problem beyond the static scratch is refused before anything runs."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(n, Nq, Nv, H, r, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    C = Nq + 2 * Nv
    dqkv = torch.randn(n, C, generator=g, device=DEV).half()
    x_q, x_v, dx_q, dx_v = (torch.randn(n, r, generator=g, device=DEV).half() for _ in range(4))
    a_q, a_v = (torch.randn(n, H, generator=g, device=DEV).half() for _ in range(2))
    return dqkv, slice(0, Nq), slice(Nq + Nv, C), x_q, x_v, a_q, a_v, dx_q, dx_v


@pytest.mark.parametrize("r", [16, 64])
def test_noalloc_equals_workspace_form(pkg, r):
    ops = pkg.ops
    Nq, Nv, H = 1536, 256, 1536
    for n, seed in ((2560, 1), (700, 2)):  # the second call smaller than the first
        print(f"lora grad noalloc r={r} n={n}", flush=True)
        args = _inputs(n, Nq, Nv, H, r, seed)
        want = ops._lora_grad(*args, 2.0)
        got = ops._lora_grad_noalloc(*args, 2.0)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b)


def test_noalloc_refuses_beyond_its_scratch(pkg):
    ops = pkg.ops
    # 64 chunks of 256 tokens x 4864 columns x rank 16 > 4 Mi fp32
    args = _inputs(64 * 256, 1536, 256, 1536, 16, 3)
    with pytest.raises(RuntimeError, match="scratch"):
        ops._lora_grad_noalloc(*args, 2.0)
