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


def test_loss_fn_kernel_matches_naive():
    from mlx_train_perf.adapters.transformers_lm import make_loss_fn

    m = _model()
    g = torch.Generator(device="cuda").manual_seed(2)
    batch = torch.randint(0, 512, (2, 65), device="cuda", generator=g)
    lengths = torch.tensor([[1, 64], [5, 40]], device="cuda")
    lk, nk = make_loss_fn(m, impl="kernel")(m, batch, lengths)
    ln, nn_ = make_loss_fn(m, impl="naive")(m, batch, lengths)
    assert int(nk) == int(nn_) and abs(lk.item() - ln.item()) < 2e-3 * abs(ln.item())


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
