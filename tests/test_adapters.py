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


def test_padding_mask_is_refused_not_ignored():
    """A left-padded batch must raise: running it as plain causal attention would silently attend to
    the padding (transformers builds no mask for a registered implementation unless asked)."""
    from mlx_train_perf.errors import AttentionInputError

    m = _tiny_llama(head_dim=64)
    x = torch.randint(0, 97, (2, 20), generator=torch.Generator().manual_seed(4))
    ref = m(input_ids=x, attention_mask=torch.ones(2, 20, dtype=torch.long)).logits
    enable_flash_attention(m, impl="reference")
    out = m(input_ids=x, attention_mask=torch.ones(2, 20, dtype=torch.long)).logits  # all ones: accepted
    assert torch.allclose(out, ref, atol=1e-4)
    padded = torch.ones(2, 20, dtype=torch.long)
    padded[1, :3] = 0
    with pytest.raises(AttentionInputError, match="padding"):
        m(input_ids=x, attention_mask=padded)
    # per-document position_ids make transformers ask for a packed mask: refused too (packed rows go
    # through mtp_segments=)
    pid = torch.cat([torch.arange(10), torch.arange(10)])[None].repeat(2, 1)
    with pytest.raises(AttentionInputError, match="non-causal"):
        m(input_ids=x, position_ids=pid, use_cache=False)


class _Rope(torch.nn.Module):
    """Rotary embedding on (B, H, L, D), the mlx-lm `nn.RoPE` convention (traditional=False)."""

    def __init__(self, dim: int, base: float = 10000.0):
        super().__init__()
        self.register_buffer("inv", base ** (-torch.arange(0, dim, 2).float() / dim), persistent=False)

    def forward(self, x):
        pos = torch.arange(x.shape[-2], dtype=torch.float32, device=x.device)
        ang = pos[:, None] * self.inv[None]
        cos, sin = ang.cos().to(x.dtype), ang.sin().to(x.dtype)
        x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
        return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)


class _MlxStyleAttention(torch.nn.Module):
    """An mlx-lm-shaped attention block (q/k/v/o_proj, rope, n_heads, n_kv_heads, scale) with the
    stock materialized causal attention."""

    def __init__(self, dim=64, n_heads=4, n_kv_heads=2, head_dim=64, seed=0):
        super().__init__()
        torch.manual_seed(seed)
        self.n_heads, self.n_kv_heads, self.scale = n_heads, n_kv_heads, head_dim ** -0.5
        self.q_proj = torch.nn.Linear(dim, n_heads * head_dim, bias=False)
        self.k_proj = torch.nn.Linear(dim, n_kv_heads * head_dim, bias=False)
        self.v_proj = torch.nn.Linear(dim, n_kv_heads * head_dim, bias=False)
        self.o_proj = torch.nn.Linear(n_heads * head_dim, dim, bias=False)
        self.rope = _Rope(head_dim)

    def forward(self, x, mask=None, cache=None):
        b, n, _ = x.shape
        q = self.rope(self.q_proj(x).reshape(b, n, self.n_heads, -1).transpose(1, 2))
        k = self.rope(self.k_proj(x).reshape(b, n, self.n_kv_heads, -1).transpose(1, 2))
        v = self.v_proj(x).reshape(b, n, self.n_kv_heads, -1).transpose(1, 2)
        rep = self.n_heads // self.n_kv_heads
        k, v = k.repeat_interleave(rep, dim=1), v.repeat_interleave(rep, dim=1)
        s = (q @ k.transpose(-1, -2)) * self.scale
        s = s.masked_fill(~torch.tril(torch.ones(n, n, dtype=torch.bool)), float("-inf"))
        o = torch.softmax(s, dim=-1) @ v
        return self.o_proj(o.transpose(1, 2).reshape(b, n, -1))


def _mlx_style_model(layers=2):
    from types import SimpleNamespace

    blocks = torch.nn.ModuleList([torch.nn.Module() for _ in range(layers)])
    for i, blk in enumerate(blocks):
        blk.self_attn = _MlxStyleAttention(seed=i)
    inner = torch.nn.Module()
    inner.layers = blocks
    model = torch.nn.Module()
    model.model = inner
    model.args = SimpleNamespace(num_attention_heads=4, num_key_value_heads=2, hidden_size=64, head_dim=64)
    return model


def test_flash_attention_wrapper_mlx_style_module():
    """enable_flash_attention on an mlx-lm-shaped model wraps each self_attn in FlashAttentionWrapper:
    the original submodules stay reachable under their names (LoRA by module path), the output matches
    the stock block, a PackedMask mask runs block-diagonal attention, and array masks / KV caches are
    refused."""
    from mlx_train_perf.attention import FlashAttentionWrapper, PackedMask
    from mlx_train_perf.attention.wrapper import is_enabled
    from mlx_train_perf.errors import AttentionInputError

    model = _mlx_style_model()
    x = torch.randn(2, 12, 64, generator=torch.Generator().manual_seed(5))
    stock = [blk.self_attn for blk in model.model.layers]
    refs = [a(x) for a in stock]
    enable_flash_attention(model, impl="reference")
    assert is_enabled(model)
    for blk, orig, ref in zip(model.model.layers, stock, refs):
        w = blk.self_attn
        assert isinstance(w, FlashAttentionWrapper)
        assert w.q_proj is orig.q_proj and w.o_proj is orig.o_proj and w.rope is orig.rope
        assert dict(w.named_parameters()).keys() == dict(orig.named_parameters()).keys()
        assert torch.allclose(w(x), ref, atol=1e-5)
        assert torch.allclose(w(x, mask="causal"), ref, atol=1e-5)
    # packed: two documents of 5 and 7 tokens; each must equal the stock block run on it alone
    # (RoPE is relative, so the second document's absolute offset does not matter)
    sid = torch.tensor([[0] * 5 + [1] * 7] * 2, dtype=torch.int32)
    sst = torch.tensor([[0] * 5 + [5] * 7] * 2, dtype=torch.int32)
    w0, orig0 = model.model.layers[0].self_attn, stock[0]
    out = w0(x, mask=PackedMask(seg_id=sid, seg_start=sst))
    assert torch.allclose(out[:, :5], orig0(x[:, :5]), atol=1e-5)
    assert torch.allclose(out[:, 5:], orig0(x[:, 5:]), atol=1e-4)
    with pytest.raises(AttentionInputError):
        w0(x, mask=torch.zeros(12, 12))
    with pytest.raises(AttentionInputError):
        w0(x, mask="sliding")
    with pytest.raises(AttentionInputError):
        w0(x, cache=object())
    enable_flash_attention(model, impl="reference")   # idempotent: no double wrapping
    assert isinstance(model.model.layers[0].self_attn.q_proj, torch.nn.Linear)
