"""C4: the 16-layer TR-GQA 200M decoder with the HIP TR-MoE layer in every
block, against the same decoder run in fp32 whose MLP halves are the oracle's
universal dispatch (engine.py:66-104 with the block's RMSNorm and residual,
block.py:270-278), fed the same bf16-rounded weights.

Prompt: 8 sequences x 2048 Zipf(1.1) token ids (C4's prefill); then 4
teacher-forced decode steps.  Bound: normwise max|got - ref| / max|ref| of
the logits <= 2e-2 (the bf16 bar), at the prefill and at every decode step.
The greedy loop's graph-replayed decode steps give the eager steps' tokens.
"""

import pytest
import torch

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu

BOUND = 2e-2


def _normwise(got, ref):
    return ((got.float() - ref.float()).abs().max() / ref.float().abs().max()).item()


def _oracle_mlp(ref_model):
    """MLP half of a block through the oracle, in fp32 on the block's weights."""
    def fn(layer, h, ids, block):
        eng = block.mlp
        p = {n: getattr(eng, n).detach() for n in ("expert_gate", "expert_up", "expert_down")}
        for n in ("shared_gate", "shared_up", "shared_down"):
            p[n] = getattr(eng, n).weight.detach()
        norm = block.post_attention_layernorm
        return O.engine_forward_norm_residual(h, ids, eng.route_table, p, norm.weight, norm.eps,
                                              route_weights=eng.config.route_weights,
                                              shared_scale=eng.config.shared_output_scale,
                                              routed_scale=eng.config.routed_output_scale)
    return fn


@pytest.fixture(scope="module")
def models(gpu):
    from complexity_amd.decoder import TRGQAConfig, TRGQADecoder

    cfg = TRGQAConfig()
    hip = TRGQADecoder(cfg).to(gpu, torch.bfloat16).init_weights(0).eval()
    ref = TRGQADecoder(cfg, backend="pytorch").to(gpu).eval()
    ref.load_state_dict({k: (v.float() if v.is_floating_point() else v) for k, v in hip.state_dict().items()})
    ref.mlp_fn = _oracle_mlp(ref)
    return hip, ref


def test_c4_prefill_and_teacher_forced_decode_match_oracle_mlp_decoder(gpu, models):
    from complexity_amd import workloads as W
    from complexity_amd.tr_hash import TRHashBackend

    hip, ref = models
    g = torch.Generator().manual_seed(0)
    ids = W.zipf_ids(8 * 2048, 32000, 1.1, g).view(8, 2048).to(gpu)
    nxt = W.zipf_ids(8 * 4, 32000, 1.1, g).view(4, 8).to(gpu)
    got = hip.prefill(ids, max_new_tokens=4)
    want = ref.prefill(ids, max_new_tokens=4)
    torch.cuda.synchronize()
    assert all(b.mlp.last_backend.selected is TRHashBackend.HIP for b in hip.layers)
    err = _normwise(got, want)
    print(f"C4 prefill logits normwise rel err {err:.3e}")
    assert err <= BOUND
    del got, want
    for s in range(4):
        got = hip.decode_step(nxt[s])
        want = ref.decode_step(nxt[s])
        err = _normwise(got, want)
        print(f"C4 decode step {s} logits normwise rel err {err:.3e}")
        assert err <= BOUND, s


def test_c4_graph_replayed_greedy_steps_equal_eager_steps(gpu, models):
    from complexity_amd import workloads as W

    hip, _ = models
    ids = W.zipf_ids(8 * 96, 32000, 1.1, torch.Generator().manual_seed(1)).view(8, 96).to(gpu)
    eager = hip.generate(ids, steps=12, use_graph=False)
    graph = hip.generate(ids, steps=12, use_graph=True)
    again = hip.generate(ids, steps=12, use_graph=True)   # a second prefill, then replays of a new capture
    torch.cuda.synchronize()
    assert torch.equal(graph, eager)
    assert torch.equal(again, eager)
