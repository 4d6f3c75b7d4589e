"""GPU: the torch integration paths run the HIP kernels end to end on a tiny bf16 Llama
(enable_flash_attention + make_loss_fn / make_packed_loss_fn), checked against eager attention and
the plain-torch loss contract."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")


def _model():
    torch.manual_seed(0)
    cfg = transformers.LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                                   max_position_embeddings=512)
    m = transformers.LlamaForCausalLM(cfg).to("cuda", torch.bfloat16).eval()
    m.config._attn_implementation = "eager"
    m.lm_head.weight.requires_grad_(False)
    return m


def test_flash_attention_kernel_matches_eager_logits():
    from mlx_train_perf.attention import enable_flash_attention
    from mlx_train_perf.attention.api import VJP_CALLS

    m = _model()
    x = torch.randint(0, 512, (2, 130), device="cuda", generator=torch.Generator(device="cuda").manual_seed(1))
    with torch.no_grad():
        ref = m(input_ids=x).logits.float()
    enable_flash_attention(m, impl="kernel", seq_len=130, batch_size=2)
    with torch.no_grad():
        out = m(input_ids=x).logits.float()
    assert float((out - ref).norm() / ref.norm()) < 2e-2
    before = VJP_CALLS.get("flash_attention_kernel_bwd", 0)
    m(input_ids=x).logits.float().sum().backward()
    assert VJP_CALLS.get("flash_attention_kernel_bwd", 0) > before


def _default_loss_by_hand(m, batch, lengths):
    """The mlx-lm trainer's `default_loss` written out independently of the adapter: the model's own
    trunk, fp64 logits against its lm_head, and the (offset, length) window walked token by token
    (inputs = batch[:, :-1], targets = batch[:, 1:], step j + 1 counted iff offset <= j + 1 <= length;
    loss = summed NLL / counted tokens)."""
    with torch.no_grad():
        hid = m.model(input_ids=batch[:, :-1]).last_hidden_state.double().cpu()
    w = m.lm_head.weight.double().cpu()
    logp = torch.log_softmax(hid @ w.T, dim=-1)
    tg = batch[:, 1:].cpu()
    total, count = 0.0, 0
    for r in range(batch.shape[0]):
        off, length = (int(x) for x in lengths[r])
        for j in range(tg.shape[1]):
            if off <= j + 1 <= length:
                total -= float(logp[r, j, tg[r, j]])
                count += 1
    return total / count, count


def test_loss_fn_kernel_matches_default_loss_by_hand():
    """make_loss_fn on the kernel impl against the documented trainer contract computed without the
    adapter (a mask or normalization bug in the adapter cannot cancel here)."""
    from mlx_train_perf.adapters.transformers_lm import make_loss_fn

    m = _model()
    g = torch.Generator(device="cuda").manual_seed(2)
    batch = torch.randint(0, 512, (3, 65), device="cuda", generator=g)
    lengths = torch.tensor([[1, 64], [5, 40], [64, 64]], device="cuda")
    want, count = _default_loss_by_hand(m, batch, lengths)
    lk, nk = make_loss_fn(m, impl="kernel")(m, batch, lengths)
    assert int(nk) == count == 64 + 36 + 1
    assert abs(lk.item() - want) < 2e-3 * abs(want), (lk.item(), want)


def test_mlx_style_wrapper_on_kernel_matches_stock():
    """FlashAttentionWrapper (the mlx-lm-shaped module surgery) with impl="kernel" on the GPU: output
    and input gradient against the stock block, computed in fp32 on the CPU; the kernel backward runs."""
    from test_adapters import _mlx_style_model

    from mlx_train_perf.attention import FlashAttentionWrapper, enable_flash_attention
    from mlx_train_perf.attention.api import VJP_CALLS

    print("[mlx-style FlashAttentionWrapper impl=kernel]", flush=True)
    stock = _mlx_style_model(layers=1).float()
    gpu = _mlx_style_model(layers=1).to("cuda", torch.bfloat16)
    x = torch.randn(2, 130, 64, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    xr = x.float().requires_grad_(True)
    ref = stock.model.layers[0].self_attn(xr)
    ref.backward(torch.ones_like(ref))
    enable_flash_attention(gpu, impl="kernel", seq_len=130, batch_size=2)
    wrap = gpu.model.layers[0].self_attn
    assert isinstance(wrap, FlashAttentionWrapper)
    xg = x.cuda().requires_grad_(True)
    before = VJP_CALLS.get("flash_attention_kernel_bwd", 0)
    out = wrap(xg, mask="causal")
    out.backward(torch.ones_like(out))
    assert VJP_CALLS.get("flash_attention_kernel_bwd", 0) == before + 1
    e_out = float((out.float().cpu() - ref.detach()).norm() / ref.detach().norm())
    e_dx = float((xg.grad.float().cpu() - xr.grad).norm() / xr.grad.norm())
    assert e_out < 2e-2 and e_dx < 3e-2, (e_out, e_dx)


def test_enable_prewarms_causal_and_packed_kernels():
    """enable_flash_attention(seq_len=, packed=True) runs the causal and the packed kernels once at the
    hinted shape (forward and backward), as the reference pre-warms its packed-keyed rate slots."""
    from mlx_train_perf.attention import enable_flash_attention
    from mlx_train_perf.attention.api import VJP_CALLS

    m = _model()
    before = VJP_CALLS.get("flash_attention_kernel_bwd", 0)
    enable_flash_attention(m, impl="kernel", seq_len=96, batch_size=2, packed=True)
    assert VJP_CALLS.get("flash_attention_kernel_bwd", 0) == before + 2
    enable_flash_attention(m, impl="kernel", seq_len=96, batch_size=2)
    assert VJP_CALLS.get("flash_attention_kernel_bwd", 0) == before + 3


def test_packed_loss_kernel_path_runs_and_matches_reference_attention():
    from mlx_train_perf.adapters.transformers_lm import make_packed_loss_fn
    from mlx_train_perf.attention import enable_flash_attention
    from mlx_train_perf.data.packing import build_row

    m = _model()
    g = torch.Generator().manual_seed(3)
    docs = [(torch.randint(1, 512, (n,), generator=g).tolist(), 1) for n in (40, 3, 70)]
    row, sid, sst, lm = build_row(docs, pack_len=128)
    args = [torch.tensor([x], device="cuda") for x in (row, sid, sst, lm)]
    enable_flash_attention(m, impl="kernel")
    lk, _ = make_packed_loss_fn(m, impl="kernel")(m, *args)
    lk.backward()
    m.zero_grad()
    m.config._mtp_flash_impl = "reference"
    lr, _ = make_packed_loss_fn(m, impl="naive")(m, *args)
    assert abs(lk.item() - lr.item()) < 2e-2 * abs(lr.item())
