"""CPU tests of the model-level API around the hot path: configuration, initialisation, loss and logits options,
precision handling, training utilities, backend selection, the torch attention functional, decoding and checkpoint
formats. They cover the behaviours the reference's own model tests check (tests/test_model_cpu.py,
tests/test_config.py, tests/test_generation.py, tests/test_checkpoint.py of tlstngud/sisa), so that a user of the
reference finds the same contract here; the numerical judge is the dense fp64 model oracle (oracle/model64.py).
"""
from __future__ import annotations

import math
import pickle
import re

import pytest
import torch
import torch.nn.functional as F

from oracle import model64 as M64
from oracle import reference as R
from model_utils import rel_err, tiny_config, tiny_model, token_ids
from sisa_amd import PRESETS, SISAAttention, SISABlock, SISAConfig, SISAForCausalLM, sisa_attention
from sisa_amd import checkpoint as CK
from sisa_amd.functional import attend_block, rotate_pairs, sisa_attention_torch
from sisa_amd.generation import SISACache

V = 257


# ------------------------------------------------------------------------------------------------ configuration
PARAMS = {"sisa-50m": 50_911_376, "sisa-152m": 151_878_576, "sisa-369m": 369_278_080}


@pytest.mark.parametrize("name", sorted(PRESETS))
def test_preset_shapes_and_counts(name):
    cfg = SISAConfig.preset(name)
    assert (cfg.d_head, cfg.d_state, cfg.vocab_size, cfg.max_seq_len) == (64, 32, 50277, 2048)
    assert cfg.n_head * cfg.d_state * 2 == cfg.d_model
    with torch.device("meta"):
        model = SISAForCausalLM(cfg)
    assert model.num_parameters() == cfg.num_parameters() == PARAMS[name]
    assert len(model.state_dict()) == 17 * cfg.n_layer + 2          # 17 tensors per block, embedding, final norm


def test_config_defaults_overrides_and_round_trip():
    assert SISAConfig() == SISAConfig.preset("sisa-50m")
    cfg = SISAConfig.preset("sisa-152m", attn_impl="torch")
    assert cfg.attn_impl == "torch" and cfg.d_model == 768
    with pytest.raises(ValueError, match="unknown preset"):
        SISAConfig.preset("sisa-7b")
    small = SISAConfig(vocab_size=99, d_model=96, n_head=3, n_layer=1, d_ff=24, d_state=6)
    assert SISAConfig.from_dict(small.to_dict()) == small
    with pytest.raises(ValueError, match="unknown SISAConfig fields"):
        SISAConfig.from_dict({**small.to_dict(), "rope_theta": 1e4})


def test_config_validation():
    with pytest.raises(ValueError, match="d_head"):
        SISAConfig(d_model=256, n_head=8, attn_impl="hip")               # d_head 32
    with pytest.raises(ValueError, match="d_state"):
        SISAConfig(d_state=16, attn_impl="hip_fused")
    SISAConfig(d_model=256, n_head=8, attn_impl="torch")
    SISAConfig(d_model=256, n_head=8, attn_impl="auto")                  # auto falls back at run time
    for bad, msg in ((dict(d_state=31, attn_impl="torch"), "even"), (dict(d_model=100, n_head=8), "divisible"),
                     (dict(attn_impl="flash"), "attn_impl"), (dict(n_layer=0), "positive"),
                     (dict(d_ff=True), "positive")):
        with pytest.raises(ValueError, match=msg):
            SISAConfig(**bad)
    assert SISAConfig().replace(attn_impl="torch").attn_impl == "torch"
    with pytest.raises(ValueError):
        SISAConfig().replace(attn_impl="nope")


def test_config_is_a_private_copy():
    cfg = tiny_config()
    model = SISAForCausalLM(cfg)
    model.set_attn_impl("auto")
    assert cfg.attn_impl == "torch" and model.config.attn_impl == "auto"
    assert model.layers[1].attn.config is model.config


# ------------------------------------------------------------------------------------------------ initialisation
def _attention_init_ok(a: SISAAttention, cfg: SISAConfig) -> None:
    assert torch.all(a.alpha_proj.bias == cfg.decay_bias_init) and torch.all(a.forget_proj.bias == cfg.forget_bias_init)
    assert torch.all(a.lambda_raw == cfg.lambda_raw_init) and a.lambda_raw.dtype == torch.float32
    assert torch.all(a.W_C.weight == 0)
    assert abs(a.theta_proj.weight.std().item() - cfg.theta_init_std) < 1e-3
    for lin in (a.W_Q, a.W_K, a.W_V, a.W_O, a.W_B, a.alpha_proj, a.forget_proj):
        assert abs(lin.weight.std().item() - cfg.init_std) < 2e-3


def test_initialisation_values():
    torch.manual_seed(0)
    cfg = tiny_config(d_model=256, n_head=4, d_ff=512)
    assert (cfg.decay_bias_init, cfg.forget_bias_init, cfg.lambda_raw_init) == (-5.0, 4.0, -1.0)
    model = SISAForCausalLM(cfg)
    for layer in model.layers:
        _attention_init_ok(layer.attn, cfg)
        for lin in (layer.ffn.w_gate, layer.ffn.w_up, layer.ffn.w_down):
            assert abs(lin.weight.std().item() - 0.02) < 2e-3
        assert torch.all(layer.attn_norm.weight == 1) and torch.all(layer.ffn_norm.weight == 1)
    assert abs(model.embed.weight.std().item() - 0.02) < 1e-3 and torch.all(model.final_norm.weight == 1)
    assert torch.allclose(model.layers[0].attn.lam(), torch.full((4,), math.log1p(math.exp(-1.0))))
    # standalone modules get the same initialisation
    _attention_init_ok(SISAAttention(cfg), cfg)
    _attention_init_ok(SISABlock(cfg).attn, cfg)
    # reset_parameters undoes a perturbation
    pert = tiny_model(seed=1, d_model=256, n_head=4, d_ff=512)
    pert.reset_parameters()
    for layer in pert.layers:
        _attention_init_ok(layer.attn, pert.config)
        assert torch.all(layer.ffn_norm.weight == 1)
    assert not torch.all(SISAForCausalLM(tiny_config(zero_init_c=False)).layers[0].attn.W_C.weight == 0)


def test_zero_c_init_is_forgetting_attention():
    """With W_C = 0 the state-space term vanishes: lambda = 0 gives bitwise the same logits."""
    torch.manual_seed(0)
    model = SISAForCausalLM(tiny_config())
    ids = token_ids(2, 40)
    ref = model(ids).logits
    with torch.no_grad():
        for layer in model.layers:
            layer.attn.lambda_raw.fill_(float("-inf"))             # softplus(-inf) = 0 exactly
    assert torch.equal(model.layers[0].attn.lam(), torch.zeros(2)) and torch.equal(model(ids).logits, ref)


# ------------------------------------------------------------------------------------------------ causality, blocks
def _first_divergent_position(a: torch.Tensor, b: torch.Tensor) -> int:
    """The first time index at which two (B, T, V) logits tensors differ anywhere (T if they never do)."""
    same = (a == b).flatten(2).all(-1).all(0)
    return int((~same).nonzero()[0]) if bool((~same).any()) else a.shape[1]


@pytest.mark.parametrize("block_q", [5, 16, 256])
def test_logits_never_see_later_tokens(block_q):
    """Replacing every token from position t on (each by a different token) changes nothing before t, bitwise, and
    changes position t itself -- for cuts inside, at the edge of and across the torch path's query blocks."""
    model = tiny_model(torch_block_q=block_q)
    ids = token_ids(2, 48, seed=11)
    base = model(ids).logits
    for t in (0, 1, block_q - 1, block_q, 47):
        if t >= ids.shape[1]:
            continue
        other = ids.clone()
        other[:, t:] = (ids[:, t:] * 31 + 5) % V
        assert bool((other[:, t:] != ids[:, t:]).all())
        assert _first_divergent_position(model(other).logits, base) == t, f"cut {t}"


def test_prefix_runs_and_block_sizes_agree():
    """Running a prefix of the sequence, or the torch path with any query-block size, evaluates the same function:
    agreement to fp32 summation-order level (1e-5 norm-wise)."""
    model = tiny_model(seed=4)
    ids = token_ids(3, 66, seed=4)
    full = model(ids).logits
    for n in (1, 17, 64, 65):
        assert rel_err(model(ids[:, :n]).logits, full[:, :n]) < 1e-5, f"prefix {n}"
    for block_q in (3, 9, 40, 1000):
        model.config.torch_block_q = block_q
        assert rel_err(model(ids).logits, full) < 1e-5, f"block_q {block_q}"


# ------------------------------------------------------------------------------------------------ loss options
def test_loss_and_logits_options():
    model = tiny_model()
    ids = token_ids(2, 33)
    out = model(ids, labels=ids)
    assert out.logits.shape == (2, 33, V) and out.logits.dtype == torch.float32 and out.loss.dim() == 0
    assert torch.equal(out.loss, F.cross_entropy(out.logits[:, :-1].reshape(-1, V), ids[:, 1:].reshape(-1)))
    with pytest.raises(ValueError, match="GPU"):
        model(ids, labels=ids, fused_ce=True)
    no_labels = model(ids, fused_ce=True)                           # fused_ce without labels: plain logits
    assert no_labels.loss is None and torch.equal(no_labels.logits, model(ids).logits)


# ------------------------------------------------------------------------------------------------ precision
def test_cpu_autocast_keeps_fp32_parameters_and_gradients():
    model = tiny_model()
    ids = token_ids(2, 24)
    ref = model(ids, labels=ids).loss
    with torch.autocast("cpu", dtype=torch.bfloat16):
        out = model(ids, labels=ids)
    assert out.logits.dtype == torch.bfloat16 and abs(out.loss.item() - ref.item()) < 2e-2
    out.loss.backward()
    for name, p in model.named_parameters():
        assert p.grad is not None and p.grad.dtype == torch.float32 and torch.isfinite(p.grad).all(), name
    assert all(layer.attn.lambda_raw.dtype == torch.float32 for layer in model.layers)


def test_lambda_raw_survives_low_precision_casts():
    model = tiny_model()
    attn = model.layers[0].attn
    with torch.no_grad():
        attn.lambda_raw.fill_(-1.0 / 3.0)
    attn.lambda_raw.grad = torch.full_like(attn.lambda_raw, 1.0 / 3.0)
    value, grad = attn.lambda_raw.detach().clone(), attn.lambda_raw.grad.clone()
    for dtype in (torch.bfloat16, torch.float16):
        model.to(dtype)
        assert attn.W_Q.weight.dtype == dtype and attn.lambda_raw.dtype == torch.float32
        assert torch.equal(attn.lambda_raw.detach(), value) and torch.equal(attn.lambda_raw.grad, grad)
    model.float()
    assert torch.equal(attn.lambda_raw.detach(), value)
    low = tiny_model().to(torch.bfloat16)
    ids = token_ids(1, 12)
    out = low(ids, labels=ids)
    assert out.logits.dtype == torch.bfloat16 and torch.isfinite(out.loss)
    low.double()
    assert low.layers[0].attn.lambda_raw.dtype == torch.float64             # only 16-bit casts are refused
    assert tiny_model().double()(token_ids(1, 10)).logits.dtype == torch.float64


# ------------------------------------------------------------------------------------------------ training utilities
def test_checkpointed_blocks_reproduce_loss_and_gradients():
    """Recomputing each block in the backward (gradient checkpointing) gives the same loss bitwise and the same
    gradients for every parameter up to reassociation (flattened vector, 1e-6 norm-wise)."""
    ids = token_ids(2, 30, seed=6)
    plain = tiny_model(seed=6).train()
    ckpt = tiny_model(seed=6, gradient_checkpointing=True).train()
    ckpt.load_state_dict(plain.state_dict())
    losses, flat = [], []
    for m in (plain, ckpt):
        loss = m(ids, labels=ids).loss
        loss.backward()
        losses.append(loss.detach())
        flat.append(torch.cat([p.grad.flatten() for _, p in sorted(m.named_parameters())]))
    assert torch.equal(losses[0], losses[1])
    assert rel_err(flat[1], flat[0]) < 1e-6


def test_parameter_counts_and_compile_common():
    model = tiny_model()
    cfg = model.config
    assert model.num_parameters() == cfg.num_parameters()
    assert model.num_parameters(exclude_embeddings=True) == cfg.num_parameters() - cfg.vocab_size * cfg.d_model
    keys = list(model.state_dict())
    assert model.compile_common() is model and list(model.state_dict()) == keys
    groups = model.param_groups(lr=6e-4, weight_decay=0.1)
    torch.optim.AdamW(groups, betas=(0.9, 0.95))
    ids = [id(p) for g in groups for p in g["params"]]
    assert len(ids) == len(set(ids)) == len(list(model.parameters()))
    assert all(p.dtype == torch.float32 for g in groups if g["name"] == "lambda" for p in g["params"])


# ------------------------------------------------------------------------------------------------ backend selection
def test_backend_selection_on_cpu():
    model = tiny_model(attn_impl="auto")
    ids = token_ids(1, 9)
    assert torch.equal(model(ids).logits, tiny_model()(ids).logits)        # auto is the torch path on the CPU
    for impl in ("hip", "hip_fused"):
        model.set_attn_impl(impl)
        with pytest.raises(ValueError, match="GPU"):
            model(ids)
    with pytest.raises(ValueError):
        model.set_attn_impl("flash")
    with pytest.raises(ValueError, match="d_head"):
        SISAForCausalLM(tiny_config(d_model=64, n_head=2)).set_attn_impl("hip")
    attn = tiny_model(attn_impl="auto").layers[0].attn
    x = torch.randn(2, 11, 128)
    assert torch.equal(attn(x, impl="torch"), attn(x))


# ------------------------------------------------------------------------------------------------ torch functional
def _dense64(q, k, v, c, b, g, lam, f):
    """The oracle's dense evaluation of the SISA formula in float64 (oracle/reference.py: dense_attention)."""
    to64 = (lambda t: None if t is None else t.detach().double())  # noqa: E731
    return R.dense_attention(*(to64(t) for t in (q, k, v, c, b, g, lam, f)))


def _inputs(seed, bsz=1, h=2, L=300, d=64, s=32, with_f=True):
    """Seeded attention inputs: unit normal q/k/v/c/b, g from log-decays -softplus(N(-2, 1)), lambda on a grid in
    [0.2, 1.4], F from log-forget gates logsigmoid(N(2, 1))."""
    gen = torch.Generator().manual_seed(100 + seed)
    normal = (lambda *shape: torch.randn(*shape, generator=gen))  # noqa: E731
    q, k, v, c, b = normal(bsz, h, L, d), normal(bsz, h, L, d), normal(bsz, h, L, d), normal(bsz, h, L, s), \
        normal(bsz, h, L, s)
    g = torch.cumsum(-F.softplus(normal(bsz, h, L) - 2.0), 2)
    lam = torch.linspace(0.2, 1.4, h)
    f = torch.cumsum(F.logsigmoid(normal(bsz, h, L) + 2.0), 2) if with_f else None
    return q, k, v, c, b, g, lam, f


@pytest.mark.parametrize("with_f", [False, True])
@pytest.mark.parametrize("shape", [(1, 1, 1, 64, 32), (1, 3, 41, 16, 8), (2, 2, 133, 64, 32), (1, 1, 90, 32, 2)])
def test_torch_attention_against_dense_fp64(shape, with_f):
    bsz, h, L, d, s = shape
    ins = _inputs(7, bsz, h, L, d, s, with_f)
    truth = _dense64(*ins)
    outs = {bq: sisa_attention_torch(*ins, block_q=bq) for bq in (1, 13, 256)}
    for bq, out in outs.items():
        assert (out.dtype, out.shape) == (torch.float32, truth.shape), bq
        assert rel_err(out, truth) < 1e-5, f"block_q {bq}: {rel_err(out, truth):.2e}"
    assert torch.equal(sisa_attention(*ins, impl="auto"), outs[256])   # auto is the torch path on the CPU


def test_torch_attention_bf16_inputs_and_gradients():
    ins = [t.bfloat16() if i < 5 else t for i, t in enumerate(_inputs(2, L=70))]
    ins = [t.requires_grad_() for t in ins]
    out = sisa_attention_torch(*ins, block_q=32)
    assert out.dtype == torch.bfloat16
    out.float().square().sum().backward()
    assert all(t.grad is not None and torch.isfinite(t.grad).all() for t in ins)


@pytest.mark.parametrize("block_q", [48, 300])
def test_torch_attention_ignores_autocast(block_q):
    """The torch path turns autocast off inside: under CPU bf16 autocast it returns exactly what it returns without
    it, for fp32 inputs (fp32 result, within 1e-5 of fp64) and for bf16 inputs (bf16 result)."""
    for cast in (None, torch.bfloat16):
        ins = list(_inputs(3, h=3, L=200))
        if cast is not None:
            ins[:5] = [t.to(cast) for t in ins[:5]]
        eager = sisa_attention_torch(*ins, block_q=block_q)
        with torch.autocast("cpu", dtype=torch.bfloat16):
            under = sisa_attention_torch(*ins, block_q=block_q)
        assert under.dtype == (cast or torch.float32) and torch.equal(under, eager)
        if cast is None:
            assert rel_err(under, _dense64(*ins)) < 1e-5


def test_decode_rows_are_fp32_under_autocast():
    q, k, v, c, b, g, lam, f = _inputs(4, L=40)
    args = ((q[:, :, -3:], c[:, :, -3:], g[:, :, -3:], f[:, :, -3:]), (k, v, b, g, f), lam, 37)
    plain = attend_block(*args)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        out = attend_block(*args)
    assert out.dtype == torch.float32
    torch.testing.assert_close(out, plain, rtol=1e-6, atol=1e-6)
    assert rel_err(out, _dense64(q, k, v, c, b, g, lam, f)[:, :, -3:]) < 1e-5


def test_torch_attention_edge_cases():
    q, c = torch.randn(1, 1, 300, 8), torch.randn(1, 1, 300, 4)
    g = torch.cumsum(torch.full((1, 1, 300), -50.0), 2)          # exp(g_i - g_j), j > i, would overflow unmasked
    assert torch.isfinite(sisa_attention_torch(q, q, q, c, c, g, torch.ones(1), None)).all()
    q, c, g, lam = torch.randn(1, 2, 5, 64), torch.randn(1, 2, 5, 32), torch.zeros(1, 2, 5), torch.ones(2)
    for impl in ("hip", "hip_fused"):
        with pytest.raises(ValueError, match=impl):
            sisa_attention(q, q, q, c, c, g, lam, impl=impl)
    with pytest.raises(ValueError):
        sisa_attention(q, q, q, c, c, g, lam, impl="other")
    with pytest.raises(ValueError):
        sisa_attention_torch(q, q, q, c, c, g, torch.ones(3))
    z, phi = torch.randn(3, 5, 8, dtype=torch.float64), torch.randn(3, 5, 4, dtype=torch.float64)
    zc = torch.view_as_complex(z.reshape(3, 5, 4, 2).contiguous()) * torch.polar(torch.ones_like(phi), phi)
    torch.testing.assert_close(rotate_pairs(z, phi), torch.view_as_real(zc).reshape(3, 5, 8))


# ------------------------------------------------------------------------------------------------ decoding
def _decoded_logits(model, ids, prompt_len, step=1):
    cache = SISACache()
    out = [model(ids[:, :prompt_len], cache=cache).logits]
    for t in range(prompt_len, ids.shape[1], step):
        out.append(model(ids[:, t:t + step], cache=cache).logits)
    assert cache.seq_len == ids.shape[1]
    return torch.cat(out, dim=1)


@pytest.mark.parametrize("prompt_len,step", [(1, 1), (5, 1), (40, 1), (7, 4)])
def test_decoding_against_full_forward_and_fp64(prompt_len, step):
    """Decode and full forward are two fp32 evaluations of one function: both are judged against fp64."""
    model = tiny_model(seed=1)
    ids = token_ids(2 if step == 1 else 1, 64 if step == 1 else 50, seed=prompt_len)
    with torch.no_grad():
        full = model(ids).logits
        dec = _decoded_logits(model, ids, prompt_len, step)
    ref = M64.logits64(model, M64.params64(model, requires_grad=False), ids)
    assert rel_err(dec, full) < 2e-5 and rel_err(dec, ref) <= 2.0 * rel_err(full, ref) + 1e-6
    assert max(rel_err(dec[:, t], full[:, t]) for t in range(ids.shape[1])) < 1e-4


def test_greedy_generation_equals_the_uncached_argmax_loop():
    model = tiny_model(seed=3)
    prompt = token_ids(2, 6, seed=3)
    out = model.generate(prompt, max_new_tokens=10)
    seq = prompt
    with torch.no_grad():
        for _ in range(10):
            seq = torch.cat([seq, model(seq).logits[:, -1].argmax(-1, keepdim=True)], dim=1)
    assert out.shape == (2, 16) and torch.equal(out, seq) and torch.equal(model.generate(prompt, 10), out)
    a = model.generate(prompt, 12, do_sample=True, temperature=0.8, generator=torch.Generator().manual_seed(0))
    b = model.generate(prompt, 12, do_sample=True, temperature=0.8, generator=torch.Generator().manual_seed(0))
    assert torch.equal(a, b)
    one = model.generate(prompt[0], 3)
    assert one.shape == (9,) and torch.equal(model.generate(prompt[0], 0), prompt[0])
    with pytest.raises(ValueError):
        model.generate(prompt, 2, do_sample=True, top_k=0)


def test_top_k_sampling_rule():
    """Sampling masks every logit below the k-th largest to -inf and draws from the softmax over the full vocabulary
    (src/sisa/generation.py:126-135): with the same seeded generator the draws equal that rule's draws; tokens tied at
    the k-th value stay candidates; top_k >= V and top_k = None sample from the plain softmax."""
    from sisa_amd.generation import _pick

    def rule(logits, temperature, k, gen):
        x = logits.float() / temperature
        if k is not None and k < x.shape[-1]:
            x = x.masked_fill(x < torch.topk(x, k, dim=-1).values[..., -1:], float("-inf"))
        return torch.multinomial(torch.softmax(x, -1), 1, generator=gen).squeeze(-1)

    logits = torch.randn(200, 97, generator=torch.Generator().manual_seed(5))
    for k, temp in ((1, 1.0), (5, 0.7), (96, 1.3), (97, 1.0), (500, 1.0), (None, 0.9)):
        got = _pick(logits, True, temp, k, torch.Generator().manual_seed(11))
        want = rule(logits, temp, k, torch.Generator().manual_seed(11))
        assert torch.equal(got, want), (k, temp)
    tied = torch.zeros(4000, 6)
    tied[:, 0] = 2.0                                  # one leader, then five logits tied at the 2nd value
    draws = _pick(tied, True, 1.0, 2, torch.Generator().manual_seed(2))
    assert set(draws.tolist()) == set(range(6))       # every tied token can be drawn
    assert torch.equal(_pick(tied, False, 1.0, 2, None), torch.zeros(4000, dtype=torch.int64))


def test_cache_slabs_grow_and_match_concatenation():
    """SISACache appends in place into preallocated slabs (doubling without a capacity); the state it hands out is
    the concatenation of everything appended, and earlier views keep their values after a regrowth."""
    gen = torch.Generator().manual_seed(0)
    parts = [dict(k=torch.randn(2, 3, n, 8, generator=gen), v=torch.randn(2, 3, n, 8, generator=gen),
                  b=torch.randn(2, 3, n, 4, generator=gen), g=torch.randn(2, 3, n, generator=gen),
                  fgate=torch.randn(2, 3, n, generator=gen), phi=torch.randn(2, 3, 2, generator=gen))
             for n in (5, 1, 1, 7, 1)]
    for capacity in (None, 64):
        cache = SISACache(capacity)
        first = None
        for i, p in enumerate(parts):
            st = cache.update(0, **p)
            if i == 0:
                first = st.k.clone(), st.k
        for name in ("k", "v", "b", "g", "fgate"):
            assert torch.equal(getattr(st, name), torch.cat([p[name] for p in parts], dim=2)), (capacity, name)
        assert torch.equal(st.phi, parts[-1]["phi"]) and cache.seq_len == 15 and len(cache) == 1
        assert torch.equal(first[1], first[0])             # the first state's view is unchanged
        slab = cache._slabs[0]
        assert slab.capacity == (64 if capacity else 20)   # 5 -> 10 (doubling) -> 20 on the 7-row append
    with pytest.raises(ValueError):
        SISACache(0)
    with pytest.raises(ValueError):
        SISACache().update(0, **dict(parts[0], g=torch.zeros(2, 3, 4)))


def test_cache_keeps_autograd_history():
    """Appends that carry autograd history are concatenated out of place, so gradients reach every appended part."""
    a = torch.randn(1, 1, 3, 4, requires_grad=True)
    b = torch.randn(1, 1, 2, 4, requires_grad=True)
    z = dict(v=torch.zeros(1, 1, 3, 4), b=torch.zeros(1, 1, 3, 2), g=torch.zeros(1, 1, 3), fgate=torch.zeros(1, 1, 3),
             phi=torch.zeros(1, 1, 1))
    cache = SISACache()
    cache.update(0, k=a, **z)
    st = cache.update(0, k=b, **{n: t[:, :, :2] if n != "phi" else t for n, t in z.items()})
    st.k.sum().backward()
    assert torch.equal(a.grad, torch.ones_like(a)) and torch.equal(b.grad, torch.ones_like(b))


def test_top_k_sampling_stays_among_the_k_largest():
    from sisa_amd.generation import _pick
    gen = torch.Generator().manual_seed(5)
    logits = torch.randn(64, 100, generator=gen)
    top3 = logits.topk(3, dim=-1).indices
    for _ in range(5):
        tok = _pick(logits, True, 0.7, 3, gen)
        assert bool((tok[:, None] == top3).any(-1).all())
    assert torch.equal(_pick(logits, False, 1.0, None, None), logits.argmax(-1))
    assert torch.equal(_pick(logits, True, 1.0, 1, gen), logits.argmax(-1))


def test_cpu_autocast_decoding_close_to_full_forward():
    model = tiny_model(seed=7)
    ids = token_ids(1, 30, seed=7)
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        full = model(ids).logits.float()
        dec = _decoded_logits(model, ids, 10).float()
    assert rel_err(dec, full) < 2e-2


# ------------------------------------------------------------------------------------------------ checkpoints
_FLAT = re.compile(r"^layers\.(\d+)\.attn\.")
_COMPILED = re.compile(r"^(layers\.\d+\.(?:attn_norm|ffn_norm|ffn)|final_norm)\.")


def _paper_layout(model, prefix=""):
    """The weights with the paper training code's key layout: flat attention keys, torch.compile's _orig_mod level
    on the compiled submodules, an optional wrapper prefix."""
    return {prefix + _COMPILED.sub(r"\1._orig_mod.", _FLAT.sub(r"layers.\1.", k)): v.clone()
            for k, v in model.state_dict().items()}


@pytest.mark.parametrize("prefix", ["", "module.", "_orig_mod.", "module._orig_mod."])
def test_paper_layout_round_trip(prefix):
    src = tiny_model(seed=1)
    conv = CK.convert_state_dict(_paper_layout(src, prefix))
    assert set(conv) == set(src.state_dict()) and CK.convert_state_dict(conv).keys() == conv.keys()
    dst = SISAForCausalLM(CK.infer_config_from_state_dict(conv, attn_impl="torch"))
    dst.load_state_dict(conv, strict=True)
    ids = token_ids(2, 20)
    assert torch.equal(dst(ids).logits, src(ids).logits)


def test_infer_config_from_shapes():
    src = tiny_model(seed=2, d_ff=200, n_layer=3)
    cfg = CK.infer_config_from_state_dict(_paper_layout(src))
    for field in ("vocab_size", "d_model", "n_layer", "n_head", "d_ff", "d_state"):
        assert getattr(cfg, field) == getattr(src.config, field), field
    with pytest.raises(ValueError, match="cannot be overridden"):
        CK.infer_config_from_state_dict(_paper_layout(src), d_ff=100)
    with pytest.raises(ValueError, match="does not describe a SISA model"):
        CK.infer_config_from_state_dict({"embed.weight": torch.zeros(3, 4)})


class _RunConfig:
    """A training-config object pickled into a checkpoint (not a tensor or plain container)."""

    lr = 3e-4


def test_paper_checkpoint_files(tmp_path):
    src = tiny_model(seed=3)
    ids = token_ids(2, 20)
    torch.save({"model": _paper_layout(src), "optimizer": {"state": {}, "param_groups": []}, "step": 7,
                "config": {"d_ff": 2048, "run_name": "x"}}, tmp_path / "final.pt")
    model = CK.load_paper_checkpoint(tmp_path / "final.pt", attn_impl="torch")
    assert not model.training and model.config.d_ff == src.config.d_ff and isinstance(model.config, SISAConfig)
    assert torch.equal(model(ids).logits, src(ids).logits)
    bf16 = CK.load_paper_checkpoint(tmp_path / "final.pt", dtype=torch.bfloat16)
    assert bf16.embed.weight.dtype == torch.bfloat16 and bf16.layers[0].attn.lambda_raw.dtype == torch.float32
    torch.save(_paper_layout(src), tmp_path / "plain.pt")                       # a bare state dict
    assert torch.equal(CK.load_paper_checkpoint(tmp_path / "plain.pt", attn_impl="torch")(ids).logits,
                       src(ids).logits)
    torch.save({"model": _paper_layout(src), "config": _RunConfig()}, tmp_path / "objs.pt")
    with pytest.raises(pickle.UnpicklingError, match="trust_pickle"):
        CK.load_paper_checkpoint(tmp_path / "objs.pt")
    trusted = CK.load_paper_checkpoint(tmp_path / "objs.pt", trust_pickle=True, attn_impl="torch")
    assert torch.equal(trusted(ids).logits, src(ids).logits)


def test_checkpoint_mismatches_raise(tmp_path):
    src = tiny_model(seed=6)
    cases = {"missing": lambda sd: sd.pop("layers.1.forget_proj.bias"),
             "unexpected": lambda sd: sd.__setitem__("layers.0.extra.weight", torch.zeros(1)),
             "shape mismatch": lambda sd: sd.__setitem__("layers.1.ffn._orig_mod.w_up.weight", torch.zeros(10, 128))}
    for msg, edit in cases.items():
        sd = _paper_layout(src)
        edit(sd)
        torch.save({"model": sd}, tmp_path / "ck.pt")
        with pytest.raises(ValueError, match=msg):
            CK.load_paper_checkpoint(tmp_path / "ck.pt")
    torch.save({"something": 1}, tmp_path / "bad.pt")
    with pytest.raises(ValueError, match="state dict"):
        CK.load_paper_checkpoint(tmp_path / "bad.pt")


def test_pretrained_directories(tmp_path):
    src = tiny_model(seed=7)
    ids = token_ids(2, 20)
    src.save_pretrained(tmp_path)
    loaded = SISAForCausalLM.from_pretrained(tmp_path)
    assert loaded.config == src.config and not loaded.training and torch.equal(loaded(ids).logits, src(ids).logits)
    other = SISAForCausalLM.from_pretrained(tmp_path, attn_impl="auto", dtype=torch.bfloat16)
    assert other.config.attn_impl == "auto" and other.embed.weight.dtype == torch.bfloat16
    with pytest.raises(ValueError, match="expects the directory save_pretrained writes"):
        SISAForCausalLM.from_pretrained(tmp_path / "missing")
    (tmp_path / "model.safetensors").unlink()
    with pytest.raises(FileNotFoundError):
        SISAForCausalLM.from_pretrained(tmp_path)


def test_parameter_manifest_is_the_state_dict():
    """SISAConfig.parameter_shapes names every tensor of the model's state dict with its shape."""
    cfg = SISAConfig(vocab_size=99, d_model=96, n_head=3, n_layer=2, d_ff=40, d_state=6)
    model = SISAForCausalLM(cfg)
    assert {k: tuple(v.shape) for k, v in model.state_dict().items()} == cfg.parameter_shapes()
    assert cfg.num_parameters() == model.num_parameters()
