"""GPU parity of the audit's margin helpers (code_for_iclr27_amd.vjp, HIP kernels through the C
ABI) against the f64 oracle: head logits for bf16/f16/f32 weights with and without bias, 1..8
rows (several row passes), odd vocabulary sizes and the Llama-3.2-1B / 3.1-8B / Qwen-style hidden
sizes; margins with given and argmax targets; hidden gradients (single target and per-row
targets with due flags); per-layer pre-projection gradients with and without the output gate.

Tolerance (f32 arithmetic, summation order differs from the reference's GEMMs): each result
within 1e-5 of the sum of the absolute values of its terms (plus 1e-6 absolute); margins and
gradients are checked on the GPU's own logits, so each kernel is checked on its own.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from code_for_iclr27_amd import vjp
from oracle import vjp as ovjp

pytestmark = pytest.mark.gpu


def model_with_head(device, vocab, dim, dtype=torch.bfloat16, bias=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    weight = (torch.randn((vocab, dim), generator=g) * 0.05).to(dtype)
    head = SimpleNamespace(weight=weight.to(device),
                           bias=(torch.randn(vocab, generator=g).to(dtype).to(device)
                                 if bias else None))
    return SimpleNamespace(get_output_embeddings=lambda: head), weight.double().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,vocab,dim,bias", [(1, 32000, 4096, False), (3, 1001, 2048, True),
                                                 (8, 4099, 4096, False), (2, 777, 5120, True)])
def test_head_logits(device, dtype, rows, vocab, dim, bias):
    model, weight = model_with_head(device, vocab, dim, dtype, bias, seed=rows)
    hidden = torch.randn((rows, dim), generator=torch.Generator().manual_seed(9))
    got = vjp.last_token_logits_float32(model, hidden.to(device).to(torch.bfloat16)).cpu().numpy()
    x = hidden.to(torch.bfloat16).double().numpy()
    b = None if not bias else model.get_output_embeddings().bias.double().cpu().numpy()
    expect = ovjp.head_logits(x, weight, b)
    scale = np.abs(x) @ np.abs(weight).T + (0 if b is None else np.abs(b))
    assert got.shape == (rows, vocab) and got.dtype == np.float32
    assert np.all(np.abs(got - expect) <= 1e-5 * scale + 1e-6)


def test_margins_given_and_argmax(device):
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal((4, 128256)) * 3).astype(np.float32)
    logits[2, 5] = logits[2, 9] = logits[2].max() + 1  # a tie: the first index wins
    dev = torch.from_numpy(logits).to(device)
    margins, targets, competitors = vjp.row_margins(dev)
    expect, expect_targets, _, _ = ovjp.margin_stats(logits)
    np.testing.assert_array_equal(targets.cpu().numpy(), expect_targets)
    assert targets[2].item() == 5
    np.testing.assert_allclose(margins.cpu().numpy(), expect, rtol=0, atol=1e-5 * (1 + np.abs(expect)).max())
    assert torch.isneginf(competitors[np.arange(4), targets]).all()
    single = vjp.one_vs_rest_margin(dev[1:2], 77)
    np.testing.assert_allclose(single.item(), ovjp.margin_stats(logits[1:2], np.array([77]))[0][0],
                               rtol=1e-6, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_hidden_gradient_single_target(device, dtype):
    vocab, dim = 32000, 4096
    model, weight = model_with_head(device, vocab, dim, dtype, seed=4)
    hidden = torch.randn((1, dim), generator=torch.Generator().manual_seed(5)).to(device)
    logits = vjp.last_token_logits_float32(model, hidden)
    target = int(logits.argmax().item())
    got = vjp.one_vs_rest_hidden_gradient(model, logits, target).cpu().numpy()
    l64 = logits.double().cpu().numpy()
    expect = ovjp.hidden_gradient(l64, np.array([target]), weight)
    comp = l64.copy()
    comp[0, target] = -np.inf
    p = np.exp(comp - comp.max()) / np.exp(comp - comp.max()).sum()
    scale = np.abs(weight[target]) + p @ np.abs(weight)
    assert got.shape == (1, dim)
    assert np.all(np.abs(got - expect) <= 1e-5 * scale + 1e-6)


def test_row_hidden_gradients_with_due(device):
    vocab, dim = 5003, 2048
    model, weight = model_with_head(device, vocab, dim, seed=6)
    logits = torch.randn((3, vocab), generator=torch.Generator().manual_seed(7)).to(device) * 2
    margins, targets, competitors = vjp.row_margins(logits)
    got = vjp.row_hidden_gradients(model, logits, targets, competitors, [True, False, True])
    got = got.cpu().numpy()
    l64 = logits.double().cpu().numpy()
    t = targets.cpu().numpy()
    expect = ovjp.hidden_gradient(l64, t, weight, np.array([1.0, 0.0, 1.0]))
    np.testing.assert_array_equal(got[1], 0.0)
    assert np.all(np.abs(got - expect) <= 1e-5 * (np.abs(weight[t]) + np.abs(weight).max()) + 1e-6)


@pytest.mark.parametrize("hidden,width,dtype,gated", [(4096, 4096, torch.bfloat16, False),
                                                      (5120, 6144, torch.bfloat16, True),
                                                      (100, 64, torch.float32, True),
                                                      (2048, 2048, torch.float16, False)])
def test_pre_gradient(device, hidden, width, dtype, gated):
    g = torch.Generator().manual_seed(hidden + width)
    o_weight = (torch.randn((hidden, width), generator=g) * 0.02).to(dtype)
    post = torch.randn(hidden, generator=g)
    gate = torch.rand(width, generator=g) if gated else None
    heads = width // 64
    got = vjp.pre_gradient(post.to(device), o_weight.to(device), heads, 64,
                           None if gate is None else gate.to(device))
    assert got.shape == (heads, 64)
    w = o_weight.double().numpy()
    expect = ovjp.pre_gradient(post.double().numpy(), w,
                               None if gate is None else gate.double().numpy())
    scale = np.abs(post.double().numpy()) @ np.abs(w)
    if gate is not None:
        scale = scale * np.abs(gate.double().numpy())
    assert np.all(np.abs(got.reshape(-1).cpu().numpy() - expect) <= 1e-5 * scale + 1e-6)


@pytest.mark.parametrize("dtype,gated", [(torch.bfloat16, False), (torch.float32, True)])
def test_pre_gradients_all_layers_match_per_layer(device, dtype, gated):
    layers, hidden, heads, dim = 5, 2048, 16, 128
    g = torch.Generator().manual_seed(21)
    weights = [(torch.randn((hidden, heads * dim), generator=g) * 0.02).to(dtype).to(device)
               for _ in range(layers)]
    posts = [torch.randn(hidden, generator=g).to(device) for _ in range(layers)]
    gates = [torch.rand(heads * dim, generator=g).to(device) if gated and l % 2 == 0 else None
             for l in range(layers)]
    batched = vjp.pre_gradients(posts, weights, heads, dim, gates)
    for l in range(layers):
        single = vjp.pre_gradient(posts[l], weights[l], heads, dim, gates[l])
        assert batched[l].shape == (heads, dim)
        torch.testing.assert_close(batched[l], single, rtol=0, atol=0)  # same kernels, same order


def test_misaligned_weight_views_rejected(device):
    hidden, heads, dim = 64, 2, 64
    backing = torch.zeros(hidden * heads * dim + 1, dtype=torch.bfloat16, device=device)
    misaligned = backing[1:].view(hidden, heads * dim)  # contiguous, 2 bytes off 16-byte alignment
    assert misaligned.data_ptr() % 16 == 2
    aligned = torch.zeros((hidden, heads * dim), dtype=torch.bfloat16, device=device)
    post = torch.ones(hidden, device=device)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        vjp.pre_gradient(post, misaligned, heads, dim)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        vjp.pre_gradients([post, post], [aligned, misaligned], heads, dim)
