"""Llama-LUCID decoder (lucid_amd.modeling_lucid): module tree, decode rows, and on the
GPU a tiny model against a float32 PyTorch reference whose attention core is the
oracle's restatement of the reference dense path.

Decode parity is defined mathematically: the V' row of a decoded token equals the row
of the same token in a prefill (P's diagonal is not 1, modeling_lucid.py:565-569)."""
import numpy as np
import pytest
import torch

from lucid_amd import modeling_lucid as M
from oracle import lucid_ref as R


def _tiny(hkv=2):
    return M.LucidConfig(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                         num_attention_heads=2, num_key_value_heads=hkv, head_dim=64)


def test_module_tree_follows_reference_names():
    torch.manual_seed(0)
    model = M.LlamaForCausalLM(_tiny())
    names = {n for n, _ in model.named_parameters()}
    for n in ("model.embed_tokens.weight", "model.layers.0.self_attn.q_proj.weight",
              "model.layers.0.self_attn.k_proj.weight", "model.layers.0.self_attn.v_proj.weight",
              "model.layers.0.self_attn.o_proj.weight", "model.layers.1.mlp.gate_proj.weight",
              "model.layers.1.mlp.up_proj.weight", "model.layers.1.mlp.down_proj.weight",
              "model.layers.1.input_layernorm.weight", "model.layers.1.post_attention_layernorm.weight",
              "model.norm.weight", "lm_head.weight"):
        assert n in names, n
    c3 = M.c3_config()
    assert (c3.num_hidden_layers, c3.hidden_size, c3.num_attention_heads, c3.head_dim, c3.intermediate_size,
            c3.vocab_size, c3.rope_theta) == (16, 2048, 32, 64, 5632, 32000, 10000.0)


@pytest.mark.parametrize("n_new", [1, 3])
def test_decode_rows_equal_prefill_rows(n_new):
    rng = np.random.default_rng(4 + n_new)
    B, H, T, d = 1, 2, 12, 16
    k = rng.standard_normal((B, H, T, d))
    v = rng.standard_normal((B, H, T, d))
    s, eps = d ** -0.5, 1e-5
    vp = R.vprime_dense(k, v, s, eps)  # prefill rows (float64 oracle)
    attn = M.LucidAttention(M.LucidConfig(hidden_size=2 * d, num_attention_heads=2, head_dim=d, rms_norm_eps=eps), 0)
    t0 = T - n_new
    kt, vt = torch.from_numpy(k), torch.from_numpy(v)
    new = attn.get_new_v_prime(kt[:, :, t0:], vt[:, :, t0:], kt[:, :, :t0], torch.from_numpy(vp[:, :, :t0]))
    np.testing.assert_allclose(new.numpy(), vp[:, :, t0:], rtol=1e-10, atol=1e-10)


def _reference_forward(model, ids, labels):
    """Run `model` with the attention core replaced by the oracle's torch restatement."""
    saved = M.lucid_attention

    def core(q, k, v, scaling=None, eps=1e-5, return_vprime=False):
        o, vp = R.lucid_attention_torch(q, k, v, scaling, eps)
        return (o, vp) if return_vprime else o

    M.lucid_attention = core
    try:
        return model(ids, labels=labels)
    finally:
        M.lucid_attention = saved


@pytest.mark.gpu
@pytest.mark.parametrize("hkv", [2, 1])
def test_tiny_model_matches_float32_reference(hkv):
    torch.manual_seed(1)
    cfg = _tiny(hkv)
    ref = M.LlamaForCausalLM(cfg)  # float32, CPU
    ours = M.LlamaForCausalLM(cfg)
    ours.load_state_dict(ref.state_dict())
    ours = ours.to("cuda", torch.bfloat16)
    T = 200
    ids = torch.randint(0, cfg.vocab_size, (1, T), generator=torch.Generator().manual_seed(2))
    print(f"case tiny model hkv={hkv} T={T}", flush=True)
    loss_ref, _ = _reference_forward(ref, ids, ids)
    loss_ref.backward()
    loss, _ = ours(ids.cuda(), labels=ids.cuda())
    loss.backward()
    torch.cuda.synchronize()
    assert abs(loss.item() - loss_ref.item()) <= 1e-2 * abs(loss_ref.item()), (loss.item(), loss_ref.item())
    assert abs(loss_ref.item() - np.log(cfg.vocab_size)) < 0.5  # random init: loss ~ ln V
    for name in ("model.layers.0.self_attn.k_proj.weight", "model.layers.1.self_attn.q_proj.weight",
                 "model.layers.0.self_attn.v_proj.weight", "model.embed_tokens.weight"):
        gr = dict(ref.named_parameters())[name].grad.double()
        go = dict(ours.named_parameters())[name].grad.double().cpu()
        cos = torch.nn.functional.cosine_similarity(gr.flatten(), go.flatten(), dim=0).item()
        rel = ((go - gr).norm() / gr.norm()).item()
        assert cos > 0.99 and rel < 0.1, (name, cos, rel)


@pytest.mark.gpu
def test_fused_layers_model_matches_float32_reference():
    """A decoder wide and long enough to take every fused path (hidden 512: the fused RMSNorm;
    B T hidden >= 2^20: the stacked q/k/v GEMM with the fused split + rotary step; the fused
    SwiGLU gate and loss) against the float32 reference model on the CPU, loss and gradients."""
    torch.manual_seed(7)
    cfg = M.LucidConfig(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                        num_attention_heads=8, num_key_value_heads=2, head_dim=64)
    ref = M.LlamaForCausalLM(cfg)  # float32, CPU
    ours = M.LlamaForCausalLM(cfg)
    ours.load_state_dict(ref.state_dict())
    ours = ours.to("cuda", torch.bfloat16)
    T = 2048
    assert T * cfg.hidden_size >= M._STACKED_QKV_MIN_NUMEL
    ids = torch.randint(0, cfg.vocab_size, (1, T), generator=torch.Generator().manual_seed(8))
    print(f"case fused-layer model T={T}", flush=True)
    loss_ref, _ = _reference_forward(ref, ids, ids)
    loss_ref.backward()
    loss, _ = ours(ids.cuda(), labels=ids.cuda())
    loss.backward()
    torch.cuda.synchronize()
    assert abs(loss.item() - loss_ref.item()) <= 1e-2 * abs(loss_ref.item()), (loss.item(), loss_ref.item())
    for name in ("model.layers.0.self_attn.q_proj.weight", "model.layers.1.self_attn.k_proj.weight",
                 "model.layers.0.self_attn.v_proj.weight", "model.layers.1.mlp.gate_proj.weight",
                 "model.layers.0.input_layernorm.weight", "model.norm.weight", "model.embed_tokens.weight"):
        gr = dict(ref.named_parameters())[name].grad.double()
        go = dict(ours.named_parameters())[name].grad.double().cpu()
        cos = torch.nn.functional.cosine_similarity(gr.flatten(), go.flatten(), dim=0).item()
        rel = ((go - gr).norm() / gr.norm()).item()
        assert cos > 0.99 and rel < 0.1, (name, cos, rel)


@pytest.mark.gpu
def test_decode_matches_prefill_logits():
    torch.manual_seed(3)
    cfg = _tiny(1)
    model = M.LlamaForCausalLM(cfg).to("cuda", torch.bfloat16).eval()
    T, n_new = 130, 2
    ids = torch.randint(0, cfg.vocab_size, (1, T + n_new), generator=torch.Generator().manual_seed(5)).cuda()
    print(f"case decode T={T} new={n_new}", flush=True)
    with torch.no_grad():
        _, full = model(ids)
        cache = M.LucidCache()
        _, pre = model(ids[:, :T], past_key_values=cache)
        steps = []
        for t in range(T, T + n_new):
            _, lg = model(ids[:, t:t + 1], past_key_values=cache)
            steps.append(lg)
    torch.cuda.synchronize()
    dec = torch.cat(steps, dim=1).float()
    ref = full[:, T:].float()
    err = (dec - ref).abs().max().item()
    assert err <= 2e-2 * max(1.0, ref.abs().max().item()), err
    assert cache.get_seq_length() == T + n_new


@pytest.mark.gpu
@pytest.mark.parametrize("heads,hkv,head_dim", [(2, 1, 64), (4, 1, 68)])
def test_decode_several_tokens_in_one_call_matches_prefill_logits(heads, hkv, head_dim):
    """Prefill, then five new tokens in one forward call (one decoding call per layer): the
    logits equal those of the whole sequence in one prefill.  head_dim 68 is the reference
    model's (lucid/config/config.json:9)."""
    torch.manual_seed(4)
    cfg = M.LucidConfig(vocab_size=512, hidden_size=heads * head_dim, intermediate_size=256, num_hidden_layers=2,
                        num_attention_heads=heads, num_key_value_heads=hkv, head_dim=head_dim)
    model = M.LlamaForCausalLM(cfg).to("cuda", torch.bfloat16).eval()
    T, n_new = 200, 5
    ids = torch.randint(0, cfg.vocab_size, (1, T + n_new), generator=torch.Generator().manual_seed(6)).cuda()
    print(f"case decode tokens model heads={heads} hkv={hkv} head_dim={head_dim}", flush=True)
    with torch.no_grad():
        _, full = model(ids)
        cache = M.LucidCache()
        model(ids[:, :T], past_key_values=cache)
        _, dec = model(ids[:, T:], past_key_values=cache)
    torch.cuda.synchronize()
    ref = full[:, T:].float()
    err = (dec.float() - ref).abs().max().item()
    assert err <= 2e-2 * max(1.0, ref.abs().max().item()), err
    assert cache.get_seq_length() == T + n_new
    assert cache.key_cache[0].shape[-1] == head_dim


def test_cache_grows_in_place_and_keeps_rows():
    cache = M.LucidCache(min_capacity=256)
    g = torch.Generator().manual_seed(7)
    k = torch.randn(2, 3, 200, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 3, 200, 64, generator=g).to(torch.bfloat16)
    kk, vv = cache.update(k, v, 0)
    assert cache.get_seq_length(0) == 200 and torch.equal(kk, k) and torch.equal(vv, v)
    kb, _, n = cache.buffers(0)
    assert kb.shape[2] == 256 and n == 200
    cache.reserve(0, k, 100)  # 300 rows > 256: doubles to 512, keeps the valid rows
    kb2, vb2, n2 = cache.buffers(0)
    assert kb2.shape[2] == 512 and n2 == 200 and torch.equal(kb2[:, :, :200], k)
    kb2[:, :, 200] = 1.0
    cache.advance(0, 1)
    assert cache.key_cache[0].shape[2] == 201 and torch.equal(cache.value_cache[0][:, :, :200], v)


@pytest.mark.gpu
def test_right_padded_batch_matches_unpadded_sequences():
    """Padded batches as the reference's data pipeline builds them (run_clm_chunk.py:517-610:
    right padding, labels -100 on padding): the real rows' logits equal those of each
    sequence alone, and the loss ignores the padding."""
    torch.manual_seed(11)
    cfg = _tiny(2)
    model = M.LlamaForCausalLM(cfg).to("cuda", torch.bfloat16).eval()
    lens, T = (70, 200), 200
    gen = torch.Generator().manual_seed(12)
    ids = torch.randint(0, cfg.vocab_size, (2, T), generator=gen)
    labels = ids.clone()
    ids[0, lens[0]:] = 0
    labels[0, lens[0]:] = -100
    print("case right-padded batch", flush=True)
    with torch.no_grad():
        loss, logits = model(ids.cuda(), labels=labels.cuda())
        for b, n in enumerate(lens):
            _, alone = model(ids[b:b + 1, :n].cuda())
            err = (logits[b, :n].float() - alone[0].float()).abs().max().item()
            assert err <= 2e-2 * max(1.0, alone.abs().max().item()), (b, err)
        # loss over the real next-token targets only
        lf = logits[:, :-1].float().reshape(-1, cfg.vocab_size)
        tgt = labels[:, 1:].reshape(-1).cuda()
        keep = tgt != -100
        ref = torch.nn.functional.cross_entropy(lf[keep], tgt[keep])
    torch.cuda.synchronize()
    assert abs(loss.item() - ref.item()) < 1e-4
