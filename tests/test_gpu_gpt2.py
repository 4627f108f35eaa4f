"""a random-init 24-layer GPT-2-medium (d 1024, 16 heads, vocab 50257, seq 1024,
batch 8) under bf16 autocast, surface "mlp+attention", rank 8, budget 0.005: one full forward,
backward and AdamW step with seeded random token ids, all 96 wrapped projections on the HIP path.

Checks: 96 layers wrapped (c_attn, attn.c_proj, c_fc, mlp.c_proj of every block); the loss equals
the unwrapped model's bit for bit (the forward is the native op); the embedding gradient (which
flows only through grad_input) matches the unwrapped model's; sampled layers' dW matches the fp64
oracle on their saved factors (fp32 weights: rel-L2 <= 1e-5); the optimizer step runs and leaves
every parameter finite.
"""
import copy

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from test_gpu_parity import _np, announce, rel_l2

pytestmark = pytest.mark.gpu

SAMPLED = ("transformer.h.0.attn.c_attn", "transformer.h.5.mlp.c_fc", "transformer.h.11.attn.c_proj",
           "transformer.h.23.mlp.c_proj")


@pytest.mark.timeout(900)
def test_config5_gpt2_medium_full_step():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    import stacr_amd
    from gpt2_tree import GPT2LMHeadModel

    dev = torch.device("cuda:0")
    announce("cfg5 build")
    torch.manual_seed(1234)
    with torch.device(dev):
        model = GPT2LMHeadModel()
    native = copy.deepcopy(model)
    layers = stacr_amd.apply_stacr(model, surface="mlp+attention", rank=8, residual_budget=0.005,
                                   turbo_after_step=None)
    assert len(layers) == 96
    names = {layer.source_name for layer in layers}
    for i in range(24):
        for leaf in ("attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj"):
            assert f"transformer.h.{i}.{leaf}" in names
    assert all(layer.transposed for layer in layers)
    stacr_amd.set_step(model, 0)

    captured = {}

    def keep(name):
        def hook(module, inputs, output):
            # the saved factors, taken now: backward frees the graph's references to them
            captured[name] = {"saved": output.grad_fn.saved_tensors, "has_residual": output.grad_fn.has_residual}
            output.register_hook(lambda g: captured[name].__setitem__("g", g.detach()))
        return hook

    for name in SAMPLED:
        model.get_submodule(name).register_forward_hook(keep(name))

    ids = torch.randint(0, 50257, (8, 1024), generator=torch.Generator(device=dev).manual_seed(7), device=dev)
    announce("cfg5 forward/backward")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss = model(ids)
        loss_native = native(ids)
    assert torch.isfinite(loss)
    assert torch.equal(loss, loss_native)
    loss.backward()
    loss_native.backward()
    wte, wte_native = model.transformer.wte.weight.grad, native.transformer.wte.weight.grad
    assert rel_l2(_np(wte), _np(wte_native)) <= 1e-3

    for name in SAMPLED:
        announce("cfg5 dW", name)
        layer = model.get_submodule(name)
        g = captured[name]["g"]
        coeff, _, q, idx, data, scale = captured[name]["saved"]
        assert coeff.dtype == torch.bfloat16 and captured[name]["has_residual"]
        rows, d_in = coeff.shape[0], layer.in_features
        oidx = idx.cpu().numpy().astype(np.int64)
        orc.check_indices(oidx, rows * d_in, ascending=True)
        vals = orc.dequantize(data.cpu().numpy().view(np.int8), np.float32(scale.item()), 8, oidx.size)
        g2d = g.reshape(rows, -1)
        odw, _ = orc.weight_grad(_np(g2d), _np(coeff), _np(q), oidx, vals, d_in)
        got = _np(layer.weight.grad).T  # Conv1D keeps (in, out)
        assert rel_l2(got, odw) <= 1e-5, name

    announce("cfg5 adamw")
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4)
    before = layers[0].weight.detach().clone()
    opt.step()
    assert not torch.equal(before, layers[0].weight)
    assert all(torch.isfinite(p).all() for p in model.parameters())
