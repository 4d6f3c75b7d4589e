"""Trainer adapter and enable_flash_attention on a tiny random-init transformers Llama (CPU).

The mlx-lm loss contract is restated here in plain torch from full logits (mask on steps in
[offset, length], sum / ntoks) -- its numerics are otherwise parity unpinned (no mlx-lm here)."""
from __future__ import annotations

import pytest
import torch

from mlx_train_perf.adapters.transformers_lm import make_loss_fn, make_packed_loss_fn, split_model
from mlx_train_perf.attention import enable_flash_attention
from mlx_train_perf.errors import AdapterError, UnsupportedAttentionError

transformers = pytest.importorskip("transformers")


def _tiny_llama(head_dim=16, tie=False, seed=0, **kw):
    torch.manual_seed(seed)
    cfg = transformers.LlamaConfig(vocab_size=97, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=head_dim,
                                   max_position_embeddings=128, tie_word_embeddings=tie, **kw)
    m = transformers.LlamaForCausalLM(cfg).eval()
    m.config._attn_implementation = "eager"
    return m


def _stock_loss(model, batch, lengths):
    inputs, targets = batch[:, :-1], batch[:, 1:]
    logits = model(input_ids=inputs).logits.float()
    ce = torch.nn.functional.cross_entropy(logits.transpose(1, 2), targets, reduction="none")
    steps = torch.arange(1, targets.shape[1] + 1)
    mask = (steps >= lengths[:, 0:1]) & (steps <= lengths[:, 1:])
    return (ce * mask).sum() / mask.sum(), mask.sum()


@pytest.mark.parametrize("impl", ["naive", "chunked"])
@pytest.mark.parametrize("tie", [False, True])
def test_make_loss_fn_matches_stock_contract(impl, tie):
    m = _tiny_llama(tie=tie)
    batch = torch.randint(0, 97, (3, 13), generator=torch.Generator().manual_seed(1))
    lengths = torch.tensor([[1, 12], [3, 9], [2, 12]])
    loss, ntoks = make_loss_fn(m, impl=impl)(m, batch, lengths)
    ref, rtoks = _stock_loss(m, batch, lengths)
    assert int(ntoks) == int(rtoks) and abs(loss.item() - ref.item()) < 1e-5
    loss.backward()
    assert m.model.layers[0].self_attn.q_proj.weight.grad is not None


def test_split_model_refusals():
    with pytest.raises(AdapterError):
        split_model(torch.nn.Linear(2, 2))
    m = _tiny_llama()
    _, head = split_model(m)
    assert head.trainable and head.weight is m.lm_head.weight


def test_enable_flash_attention_reference_matches_eager():
    m = _tiny_llama(head_dim=64)
    x = torch.randint(0, 97, (2, 20), generator=torch.Generator().manual_seed(2))
    ref = m(input_ids=x).logits
    enable_flash_attention(m, impl="reference")
    out = m(input_ids=x).logits
    assert torch.allclose(out, ref, atol=1e-4)


def test_enable_flash_attention_refusals():
    with pytest.raises(UnsupportedAttentionError):
        enable_flash_attention(_tiny_llama(head_dim=16), impl="kernel", seq_len=16)  # head_dim 16 unsupported
    with pytest.raises(UnsupportedAttentionError):
        enable_flash_attention(_tiny_llama(head_dim=64, attention_dropout=0.1))
    with pytest.raises(UnsupportedAttentionError):
        enable_flash_attention(torch.nn.Linear(2, 2))


def test_packed_loss_equals_per_document_losses():
    """RoPE depends only on relative position, so a packed row with block-diagonal attention must give
    each document the same NLL as running it alone (the reference pins packed vs unpacked at 2e-2)."""
    from mlx_train_perf.data.packing import build_row

    m = _tiny_llama(head_dim=64)
    g = torch.Generator().manual_seed(3)
    docs = [(torch.randint(1, 97, (7,), generator=g).tolist(), 1), (torch.randint(1, 97, (5,), generator=g).tolist(), 1)]
    row, sid, sst, lmask = build_row(docs, pack_len=16)
    enable_flash_attention(m, impl="reference")
    loss_fn = make_packed_loss_fn(m, impl="naive")
    loss, ntoks = loss_fn(m, torch.tensor([row]), torch.tensor([sid]), torch.tensor([sst]), torch.tensor([lmask]))
    total, count = 0.0, 0
    for tokens, off in docs:
        b = torch.tensor([tokens + [0]])
        l, n = _stock_loss(m, b, torch.tensor([[off, len(tokens) - 1 + 1]]))
        total += l.item() * int(n)
        count += int(n)
    assert int(ntoks) == count and abs(loss.item() - total / count) < 1e-4


def test_packed_loss_requires_enable():
    with pytest.raises(AdapterError):
        make_packed_loss_fn(_tiny_llama())
