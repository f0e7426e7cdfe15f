"""CPU tests of the model around the hot path: presets and parameter counts, the torch path against the dense fp64
oracle (oracle/model64.py) and the oracle's own pinning, cached decoding, checkpoint formats and the optimizer
groups. Follows the reference's CPU model tests (tests/test_config.py:6-40, tests/test_model_cpu.py,
tests/test_checkpoint.py, tests/test_generation.py of tlstngud/sisa).
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import sisa_amd as S
from oracle import model64 as M64
from sisa_amd import checkpoint as CK
from sisa_amd.generation import _eos_ids

from model_utils import perturb_, rel_err, tiny_config, tiny_model, token_ids

# parameter counts of the paper models (src/sisa/config.py:143-149, tests/test_config.py:6-10)
EXPECTED = {"sisa-50m": 50_911_376, "sisa-152m": 151_878_576, "sisa-369m": 369_278_080}


@pytest.mark.parametrize("name", sorted(EXPECTED))
def test_preset_parameter_counts(name):
    cfg = S.SISAConfig.preset(name)
    with torch.device("meta"):
        model = S.SISAForCausalLM(cfg)
    assert model.num_parameters() == EXPECTED[name] == cfg.num_parameters()
    assert len(model.state_dict()) == 2 + 17 * cfg.n_layer
    assert cfg.d_head == 64 and cfg.d_state == 32 and cfg.n_head * cfg.d_state == cfg.d_model // 2


def test_defaults_and_init():
    assert S.SISAConfig() == S.SISAConfig.preset("sisa-50m")
    torch.manual_seed(0)
    m = S.SISAForCausalLM(tiny_config())
    a = m.layers[0].attn
    assert torch.count_nonzero(a.W_C.weight) == 0                          # zero_init_c
    assert torch.all(a.alpha_proj.bias == -5.0) and torch.all(a.forget_proj.bias == 4.0)
    assert torch.all(a.lambda_raw == -1.0) and torch.all(m.final_norm.weight == 1.0)
    assert abs(float(a.theta_proj.weight.detach().std()) - 0.01) < 0.003
    m.to(torch.bfloat16)
    assert a.lambda_raw.dtype == torch.float32 and a.W_Q.weight.dtype == torch.bfloat16


def test_torch_path_matches_fp64_oracle():
    model = tiny_model(seed=1)
    ids = token_ids(2, 37, seed=1)
    loss64, logits64, grads64 = M64.loss_and_grads64(model, ids, ids)
    model.zero_grad(set_to_none=True)
    out = model(ids, labels=ids)
    out.loss.backward()
    assert abs(out.loss.item() - loss64) / loss64 < 1e-5
    assert rel_err(out.logits, logits64) < 1e-5
    for n, p in model.named_parameters():
        assert rel_err(p.grad, grads64[n]) < 2e-4, n


def test_oracle_gradcheck_tiny():
    """Finite differences of the fp64 oracle on a 1-layer model of width 16 (d_head 8, d_state 4)."""
    cfg = S.SISAConfig(vocab_size=11, d_model=16, n_layer=1, n_head=2, d_ff=24, d_state=4, attn_impl="torch")
    torch.manual_seed(3)
    model = perturb_(S.SISAForCausalLM(cfg), 3)
    ids = token_ids(1, 5, vocab=11, seed=3)
    names = [n for n, _ in model.named_parameters()]
    base = M64.params64(model, requires_grad=False)

    def f(*vals):
        P = dict(base)
        P.update(zip(names, vals))
        logits = M64.logits64(model, P, ids)
        return F.cross_entropy(logits[:, :-1].reshape(-1, 11), ids[:, 1:].reshape(-1))
    vals = [base[n].clone().requires_grad_(True) for n in names]
    assert torch.autograd.gradcheck(f, vals, eps=1e-6, atol=1e-6, rtol=1e-4)


def test_oracle_reduces_to_transformer():
    """lambda = 0 and F = 0: every layer is a pre-norm block with plain causal softmax attention."""
    model = tiny_model(seed=4)
    with torch.no_grad():
        for layer in model.layers:
            layer.attn.lambda_raw.fill_(-1e4)                  # softplus -> 0
            layer.attn.forget_proj.weight.zero_()
            layer.attn.forget_proj.bias.fill_(1e4)             # logsigmoid -> 0
    ids = token_ids(1, 23, seed=4)
    P = M64.params64(model, requires_grad=False)
    got = M64.logits64(model, P, ids)
    cfg = model.config
    x = F.embedding(ids, P["embed.weight"])
    for i in range(cfg.n_layer):
        pre = f"layers.{i}."
        n = M64._rmsnorm(x, P[pre + "attn_norm.weight"], cfg.norm_eps)
        heads = [F.linear(n, P[pre + f"attn.{w}.weight"]).view(1, 23, cfg.n_head, 64).transpose(1, 2)
                 for w in ("W_Q", "W_K", "W_V")]
        y = F.scaled_dot_product_attention(*heads, is_causal=True)
        x = x + F.linear(y.transpose(1, 2).reshape(1, 23, -1), P[pre + "attn.W_O.weight"])
        m = M64._rmsnorm(x, P[pre + "ffn_norm.weight"], cfg.norm_eps)
        x = x + F.linear(F.silu(F.linear(m, P[pre + "ffn.w_gate.weight"])) * F.linear(m, P[pre + "ffn.w_up.weight"]),
                         P[pre + "ffn.w_down.weight"])
    ref = M64._rmsnorm(x, P["final_norm.weight"], cfg.norm_eps) @ P["embed.weight"].t()
    assert rel_err(got, ref) < 1e-12


def test_cached_decoding_matches_full_forward():
    model = tiny_model(seed=5).eval()
    ids = token_ids(2, 29, seed=5)
    with torch.no_grad():
        full = model(ids).logits
        cache = S.SISACache()
        pre = model(ids[:, :17], cache=cache).logits
        steps = [pre] + [model(ids[:, t:t + 1], cache=cache).logits for t in range(17, 23)]
        steps.append(model(ids[:, 23:], cache=cache).logits)      # a multi-token step after the cache
    got = torch.cat(steps, dim=1)
    assert cache.seq_len == 29 and len(cache) == model.config.n_layer
    assert rel_err(got, full) < 1e-5


def test_generate_greedy_and_eos():
    model = tiny_model(seed=6).eval()
    ids = token_ids(2, 7, seed=6)
    out = S.generate(model, ids, 5)
    assert out.shape == (2, 12) and torch.equal(out[:, :7], ids)
    with torch.no_grad():
        full = model(out[:, :-1]).logits
    assert torch.equal(full[:, 6:].argmax(-1), out[:, 7:])        # every new token is the greedy choice
    eos = int(out[0, 7])
    stop = S.generate(model, ids, 5, eos_token_id=eos)
    assert stop[0, 7] == eos and torch.all(stop[0, 7:] == eos)    # finished rows padded with the eos id
    one = S.generate(model, ids[0], 3)
    assert one.dim() == 1 and torch.equal(one, out[0, :10])
    sampled = S.generate(model, ids, 4, do_sample=True, top_k=1, generator=torch.Generator().manual_seed(0))
    assert torch.equal(sampled, out[:, :11])                      # top_k = 1 sampling is greedy
    with pytest.raises(ValueError):
        S.generate(model, ids, -1)
    with pytest.raises(ValueError):
        S.generate(model, ids, 2, do_sample=True, temperature=0.0)


def test_eos_ids_types():
    import numpy as np
    assert _eos_ids(None) == [] and _eos_ids(3) == [3] and _eos_ids([1, 2]) == [1, 2]
    assert _eos_ids(torch.tensor(5)) == [5] and _eos_ids(torch.tensor([5, 6])) == [5, 6]
    assert _eos_ids(np.array([7, 8])) == [7, 8] and _eos_ids(np.int64(9)) == [9]
    for bad in (True, "a", 1.5, [1, 2.0], torch.tensor([1.0]), torch.zeros(2, 2, dtype=torch.long)):
        with pytest.raises(TypeError):
            _eos_ids(bad)


@pytest.mark.parametrize("safe", [True, False])
def test_save_and_load_pretrained(tmp_path, safe):
    model = tiny_model(seed=7)
    model.save_pretrained(str(tmp_path), safe_serialization=safe)
    names = sorted(p.name for p in tmp_path.iterdir())
    assert names == sorted(["config.json", "model.safetensors" if safe else "pytorch_model.bin"])
    back = S.SISAForCausalLM.from_pretrained(str(tmp_path), attn_impl="torch")
    assert not back.training and back.config == model.config
    for (n, a), (_, b) in zip(model.state_dict().items(), back.state_dict().items()):
        assert torch.equal(a, b), n
    model.save_pretrained(str(tmp_path), safe_serialization=not safe)   # the other format replaces the stale file
    assert len([p for p in tmp_path.iterdir() if p.name != "config.json"]) == 1
    with pytest.raises(ValueError):
        S.SISAForCausalLM.from_pretrained(str(tmp_path / "config.json"))


def test_paper_checkpoint_keys(tmp_path):
    """Flat attention keys, torch.compile's _orig_mod level and DDP's module. prefix map to the package layout."""
    model = tiny_model(seed=8)
    sd = model.state_dict()
    paper = {}
    for k, v in sd.items():
        k2 = k.replace(".attn.", ".")
        k2 = k2.replace(".ffn.", ".ffn._orig_mod.")
        paper["module." + k2] = v
    assert CK.convert_state_dict(paper).keys() == sd.keys()
    assert CK.convert_state_dict(sd).keys() == sd.keys()                # idempotent
    torch.save({"model": paper, "optimizer": {"step": torch.tensor(3)}, "config": {"d_ff": 999}}, tmp_path / "ck.pt")
    loaded = S.load_paper_checkpoint(tmp_path / "ck.pt", attn_impl="torch")
    assert loaded.config.d_ff == 256 and loaded.config.n_layer == 2      # shapes from the tensors, not the config
    assert all(torch.equal(loaded.state_dict()[k], v) for k, v in sd.items())
    with pytest.raises(ValueError, match="cannot be overridden"):
        CK.infer_config_from_state_dict(sd, d_model=64)
    with pytest.raises(ValueError, match="is absent"):
        CK.infer_config_from_state_dict({k: v for k, v in sd.items() if "lambda_raw" not in k})
    bad = dict(sd)
    bad["layers.0.attn.W_Q.weight"] = torch.zeros(3, 3)
    with pytest.raises(ValueError, match="shape mismatch"):
        CK.model_from_state_dict(model.config, bad)
    with pytest.raises(ValueError, match="two checkpoint keys"):
        CK.convert_state_dict({"layers.0.W_Q.weight": sd["layers.0.attn.W_Q.weight"],
                               "layers.0.attn.W_Q.weight": sd["layers.0.attn.W_Q.weight"]})


def test_param_groups():
    model = tiny_model(seed=9)
    groups = model.param_groups(1e-3, weight_decay=0.1, lambda_lr=5e-3)
    names = [g["name"] for g in groups]
    assert names == ["default", "timescale_biases", "lambda"]
    n_params = sum(len(g["params"]) for g in groups)
    assert n_params == len(list(model.parameters()))
    assert groups[2]["lr"] == 5e-3 and groups[1]["weight_decay"] == 0.0 and len(groups[2]["params"]) == 2
    flat = model.param_groups(1e-3, no_decay_timescale_biases=False)
    assert [g["name"] for g in flat] == ["default", "lambda"]


def test_loss_conventions():
    model = tiny_model(seed=10)
    ids = token_ids(2, 15, seed=10)
    labels = ids.clone()
    labels[0, 5:9] = -100
    out = model(ids, labels=labels)
    ref = F.cross_entropy(out.logits[:, :-1].reshape(-1, 257).float(), labels[:, 1:].reshape(-1), ignore_index=-100)
    assert torch.allclose(out.loss, ref)
    lossonly = model(ids, labels=labels, return_logits=False)
    assert lossonly.logits is None and torch.allclose(lossonly.loss, ref, rtol=1e-6)
    last = model(ids, logits_to_keep=3).logits
    assert last.shape == (2, 3, 257) and torch.allclose(last, out.logits[:, -3:], atol=1e-6)
    with pytest.raises(ValueError):
        model(ids, labels=labels[:, :5])
    with pytest.raises(ValueError):
        model(ids, labels=labels, logits_to_keep=2)
    with pytest.raises(ValueError, match="GPU"):
        model(ids, labels=labels, fused_ce=True)
    assert math.isfinite(out.loss.item())
