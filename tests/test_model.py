"""TinyMamba on the CPU (the reference's tests/test_model.py gates):
associative scan = recurrence (odd lengths, chunked carry), the parameter
budget and the 18M / 60M / 80M model sizes, shapes, causality, overfitting one
batch, and the recurrent cache = recomputing the whole context.
"""
from __future__ import annotations

import pytest
import torch

from mamba_metal_scan_amd.model import (MambaConfig, TinyMamba, d_inner_for_budget,
                                        mamba_block_params, parallel_scan, scan_recurrence,
                                        transformer_block_params)

SEED = 1337
VOCAB = 200


def small_cfg(**over):
    kw = dict(vocab_size=VOCAB, d_model=64, n_layers=2, d_ff=128, max_seq_len=64,
              d_state=8, d_conv=4, scan_chunk=0)
    kw.update(over)
    return MambaConfig(**kw)


def tokens(batch=4, seq=32, seed=SEED, vocab=VOCAB):
    return torch.randint(0, vocab, (batch, seq), generator=torch.Generator().manual_seed(seed))


def _pairs(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(*shape, generator=g).clamp(0.01, 0.99),
            torch.randn(*shape, generator=g))


@pytest.mark.parametrize("t_len", [1, 2, 3, 5, 17, 33, 64])
def test_parallel_scan_equals_recurrence(t_len):
    a, b = _pairs((2, t_len, 3, 5), SEED + t_len)
    assert torch.allclose(parallel_scan(a, b), scan_recurrence(a, b), atol=1e-5)


@pytest.mark.parametrize("chunk", [1, 5, 8, 40, 64])
def test_chunked_scan_carries_the_state(chunk):
    a, b = _pairs((2, 40, 7), SEED + 1)
    assert torch.allclose(parallel_scan(a, b, chunk=chunk), scan_recurrence(a, b), atol=1e-5)


def test_parameter_budget_matches_the_transformer():
    d_model, d_ff = 384, 1536
    target = transformer_block_params(d_model, d_ff)
    d_inner = d_inner_for_budget(target, d_model, 16, 4)
    assert d_inner % 8 == 0
    assert mamba_block_params(d_model, d_inner, 16, 4) <= target
    assert mamba_block_params(d_model, d_inner + 8, 16, 4) > target
    cfg = MambaConfig(vocab_size=VOCAB, d_model=d_model, n_layers=10, d_ff=d_ff, d_state=16)
    model = TinyMamba(cfg)
    expect = (VOCAB * d_model + 10 * mamba_block_params(d_model, model.d_inner, 16, 4) + d_model)
    assert model.count_params() == expect
    ours = 10 * mamba_block_params(d_model, model.d_inner, 16, 4)
    assert abs(ours - 10 * target) / (10 * target) < 0.01


@pytest.mark.parametrize("d_model,d_ff,d_state,vocab,layers,d_inner,params", [
    (384, 1536, 16, 200, 10, 856, None),            # the "18M" model
    (384, 1536, 8, 200, 10, 864, None),
    (640, 2560, 16, 200, 12, 1432, 58_682_208),     # "60M" (bench SIZES, small vocab)
    (640, 2560, 16, 32768, 12, 1432, 79_525_728),   # "80M" (vocab 32768)
])
def test_model_sizes(d_model, d_ff, d_state, vocab, layers, d_inner, params):
    target = transformer_block_params(d_model, d_ff)
    assert d_inner_for_budget(target, d_model, d_state, 4) == d_inner
    if params is not None:
        total = (vocab * d_model + layers * mamba_block_params(d_model, d_inner, d_state, 4)
                 + d_model)
        assert total == params


def test_shapes_and_dtypes():
    torch.manual_seed(SEED)
    model = TinyMamba(small_cfg())
    x = tokens()
    logits, loss = model(x, x)
    assert logits.shape == (4, 32, VOCAB) and logits.dtype == torch.float32
    assert loss.dtype == torch.float32 and loss.item() > 0
    assert model.head.weight is model.tok.weight


def test_future_tokens_do_not_leak():
    torch.manual_seed(SEED)
    model = TinyMamba(small_cfg()).eval()
    x = tokens()
    x2 = x.clone()
    x2[:, 16:] = (x2[:, 16:] + 1) % VOCAB
    with torch.no_grad():
        a, _ = model(x)
        b, _ = model(x2)
    assert torch.equal(a[:, :16], b[:, :16])
    assert not torch.allclose(a[:, 16:], b[:, 16:])


def test_torch_scan_impl_matches_the_parallel_scan():
    """scan_impl 'torch' (the T-loop reference) and 'auto' on CPU (parallel_scan)
    compute the same loss and gradients."""
    torch.manual_seed(SEED)
    m1 = TinyMamba(small_cfg(scan_impl="auto"))
    m2 = TinyMamba(small_cfg(scan_impl="torch"))
    m2.load_state_dict(m1.state_dict())
    x = tokens(batch=2, seq=24)
    _, l1 = m1(x, x)
    _, l2 = m2(x, x)
    l1.backward()
    l2.backward()
    assert torch.allclose(l1, l2, atol=1e-5)
    for (n, p1), p2 in zip(m1.named_parameters(), m2.parameters()):
        assert torch.allclose(p1.grad, p2.grad, atol=1e-5, rtol=1e-4), n


def test_overfit_one_batch():
    torch.manual_seed(SEED)
    model = TinyMamba(small_cfg())
    x = tokens()
    opt = torch.optim.AdamW(model.parameters(), lr=0.01)
    for _ in range(200):
        _, loss = model(x, x)
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
    assert loss.item() < 1.0, f"did not overfit: final loss {loss.item():.4f}"


def test_recurrent_cache_matches_full_recomputation():
    torch.manual_seed(SEED)
    model = TinyMamba(small_cfg(scan_chunk=8)).eval()
    full = tokens(seq=26)
    ctx, rest = full[:, :20], full[:, 20:]
    with torch.no_grad():
        cache: dict = {}
        model(ctx, cache=cache)
        for t in range(rest.shape[1]):
            step_logits, _ = model(rest[:, t:t + 1], cache=cache)
            assert step_logits.shape == (4, 1, VOCAB)
            full_logits, _ = model(torch.cat([ctx, rest[:, :t + 1]], dim=1))
            delta = (step_logits[:, -1] - full_logits[:, -1]).abs().max().item()
            assert delta < 1e-5, f"step {t}: cache diverges by {delta:.2e}"


def test_folded_norm_path_only_for_plain_blocks():
    """The HIP forward that folds each residual add into the next norm calls
    block.mix() instead of block(x): it is taken only for MambaBlocks that
    are neither wrapped, subclassed nor hooked, so that hooks still run."""
    from mamba_metal_scan_amd.model import MambaBlock, _plain_block
    model = TinyMamba(small_cfg())
    assert all(_plain_block(b) for b in model.blocks)
    h = model.blocks[0].register_forward_hook(lambda *a: None)
    assert not _plain_block(model.blocks[0]) and _plain_block(model.blocks[1])
    h.remove()
    assert _plain_block(model.blocks[0])

    class Sub(MambaBlock):
        pass

    assert not _plain_block(Sub(small_cfg(), model.blocks[0].d_inner))
    assert not _plain_block(torch.nn.Sequential(model.blocks[0]))
    g = torch.nn.modules.module.register_module_forward_hook(lambda *a: None)
    try:
        assert not _plain_block(model.blocks[1])
    finally:
        g.remove()
