"""q36moe_forward_noalloc (the layer on the library's static per-GPU
scratch, for callers that cannot allocate) against q36moe_forward on a
context: bit-identical outputs on two calls in a row, the second smaller,
on the sorted and direct paths, with and without the shared expert; sizes
past its maximum are refused."""
import numpy as np
import pytest
import torch

from q36_amd import moe, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def weights():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    w = synth.expert_weights(2101, shared=True)
    return moe.MoEWeights.upload(w["gate"], w["up"], w["down"], w["sh_gate"], w["sh_up"], w["sh_down"])


def _inputs(rng, T, shared):
    dev = torch.device("cuda:0")
    x = torch.from_numpy(synth.hidden(rng, T)).to(dev)
    lg = torch.from_numpy(synth.normal_logits(rng, T)).to(dev)
    shg = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).to(dev) if shared else None
    return x, lg, shg


@pytest.mark.parametrize("sizes,shared", [((40, 5), False), ((64, 33), True), ((16, 1), True)])
def test_noalloc_equals_forward(weights, sizes, shared):
    rng = np.random.default_rng(2200 + sizes[0] + sizes[1])
    for T in sizes:   # two calls in a row on the same static scratch, the second smaller
        x, lg, shg = _inputs(rng, T, shared)
        out = torch.full((T, 2048), float("nan"), dtype=torch.float32, device="cuda:0")
        moe.forward_noalloc(weights, x, lg, shg, out=out)
        ref = moe.MoELayer(T).forward(weights, x, lg, shg, out_dtype=torch.float32)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), ref.cpu().numpy())
        ob = moe.forward_noalloc(weights, x, lg, shg, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        assert torch.equal(ob, ref.to(torch.bfloat16))


def test_noalloc_refuses_past_max(weights):
    x, lg, _ = _inputs(np.random.default_rng(2300), moe.NOALLOC_MAX_T + 1, False)
    with pytest.raises(moe.Q36MoEError):
        moe.forward_noalloc(weights, x, lg)
    e = torch.zeros((0, 2048), device="cuda:0")
    assert moe.forward_noalloc(weights, e, torch.zeros((0, 256), device="cuda:0")).shape == (0, 2048)
