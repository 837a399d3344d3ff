"""The TR-GQA decoder harness on the CPU (fp32, the universal MLP path):
RoPE tables against their closed form, the grouped decode attention against
repeat_interleave + SDPA (gqa.py:150-152), and the static KV cache: a prompt
prefilled then extended by decode steps gives the logits of the longer
prompt prefilled at once."""

import math

import pytest
import torch
import torch.nn.functional as F

from complexity_amd.decoder import TRGQAConfig, TRGQADecoder, rope_tables

SMALL = TRGQAConfig(vocab_size=211, hidden_size=64, num_layers=2, num_heads=6, num_kv_heads=2, head_dim=16,
                    shared_width=48, num_experts=4, expert_width=8, max_position_embeddings=32)


def _model(cfg=SMALL, seed=0):
    torch.manual_seed(0)
    return TRGQADecoder(cfg, backend="pytorch").init_weights(seed).eval()


def test_rope_tables_closed_form():
    D, theta = 16, 10000.0
    cos, sin = rope_tables(D, 40, theta)
    for p in (0, 1, 7, 39):
        for i in range(D):
            ang = p * theta ** (-2.0 * (i % (D // 2)) / D)
            assert cos[p, i].item() == pytest.approx(math.cos(ang), abs=1e-5)
            assert sin[p, i].item() == pytest.approx(math.sin(ang), abs=1e-5)


def test_grouped_decode_attention_equals_repeated_heads():
    torch.manual_seed(1)
    m = _model()
    attn = m.layers[0].self_attn
    B, L, D = 3, 20, SMALL.head_dim
    q = torch.randn(B, SMALL.num_heads, 1, D)
    k = torch.randn(B, SMALL.num_kv_heads, L, D)
    v = torch.randn(B, SMALL.num_kv_heads, L, D)
    pos = 13
    mask = torch.where(torch.arange(L) <= pos, 0.0, -1e9).view(1, 1, 1, L)
    got = attn.decode_attention(q, k, v, mask)
    kr = k[:, :, :pos + 1].repeat_interleave(SMALL.kv_groups, dim=1)
    vr = v[:, :, :pos + 1].repeat_interleave(SMALL.kv_groups, dim=1)
    want = F.scaled_dot_product_attention(q, kr, vr, scale=1.0 / math.sqrt(D))
    assert torch.allclose(got, want, atol=1e-5, rtol=1e-5)


def test_prefill_then_decode_matches_longer_prefill():
    m = _model()
    ids = torch.randint(0, SMALL.vocab_size, (2, 11), generator=torch.Generator().manual_seed(3))
    full = m.prefill(ids)                       # [2, 11, V]
    part = m.prefill(ids[:, :8], max_new_tokens=3)
    assert torch.allclose(part, full[:, :8], atol=1e-5, rtol=1e-5)
    for t in range(8, 11):
        step = m.decode_step(ids[:, t])
        assert torch.allclose(step, full[:, t], atol=1e-4, rtol=1e-4), t


def test_greedy_generate_eager_is_argmax_of_decode():
    m = _model()
    ids = torch.randint(0, SMALL.vocab_size, (2, 5), generator=torch.Generator().manual_seed(4))
    toks = m.generate(ids, steps=4, use_graph=False)
    assert toks.shape == (2, 5)
    seq = ids
    for s in range(5):
        nxt = m.prefill(seq)[:, -1].argmax(-1)
        assert torch.equal(nxt, toks[:, s]), s
        seq = torch.cat([seq, nxt[:, None]], dim=1)


def test_init_weights_is_seeded_and_scales_residual_projections():
    a, b = _model(seed=7), _model(seed=7)
    for (n, p), (_, q) in zip(a.named_parameters(), b.named_parameters()):
        assert torch.equal(p, q), n
    cfg = TRGQAConfig(vocab_size=100, hidden_size=256, num_layers=8, num_heads=4, num_kv_heads=2, head_dim=64,
                      shared_width=512, num_experts=4, expert_width=64)
    m = TRGQADecoder(cfg, backend="pytorch").init_weights(1)
    std = cfg.initializer_range
    res = std / math.sqrt(2 * cfg.num_layers)
    blk = m.layers[3]
    assert blk.self_attn.q_proj.weight.std().item() == pytest.approx(std, rel=0.05)
    assert blk.self_attn.o_proj.weight.std().item() == pytest.approx(res, rel=0.05)
    assert blk.mlp.shared_down.weight.std().item() == pytest.approx(res, rel=0.05)
    assert blk.mlp.expert_down.std().item() == pytest.approx(res, rel=0.05)
    assert blk.mlp.shared_gate.weight.std().item() == pytest.approx(std, rel=0.05)
    assert torch.equal(blk.post_attention_layernorm.weight, torch.ones(cfg.hidden_size))
    # each layer routes with its own table (routing.py layer salt)
    assert not torch.equal(m.layers[0].mlp.route_table, m.layers[1].mlp.route_table)
    assert m.layers[5].mlp.config.layer_index == 5
