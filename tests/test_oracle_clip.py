"""Pinning the CLIP text-encoder oracle (oracle/clip_ref.py) on the CPU.

The reference's text encoder is a LiteRT export of SD1.5's ``CLIPTextModel``
(VulkanUnetPipeline.kt:48-53); no weights or encoded fixtures ship with it.  The
restatement is pinned against transformers' own ``CLIPTextModel`` (the published
implementation, importable offline) built from the same configuration and loaded with
the same seeded weights, and planted mistakes (no causal mask, exact GELU for
quick-GELU, post-LayerNorm) must each fail that comparison.
"""
import numpy as np
import pytest
import torch

from oracle import clip_ref

transformers = pytest.importorskip("transformers")


def _hf_model(p, vocab, hidden, layers, heads, ffn):
    cfg = transformers.CLIPTextConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=ffn,
                                      num_hidden_layers=layers, num_attention_heads=heads,
                                      max_position_embeddings=clip_ref.SEQ, hidden_act="quick_gelu",
                                      layer_norm_eps=clip_ref.EPS, bos_token_id=0, eos_token_id=1,
                                      pad_token_id=1)
    m = transformers.CLIPTextModel(cfg).eval()
    keys = m.state_dict().keys()
    sd = {}
    for k in keys:
        src = k if k in p else clip_ref.PREFIX + (k[len("text_model."):] if k.startswith("text_model.") else k)
        if src not in p:
            continue  # e.g. position_ids buffers
        sd[k] = torch.as_tensor(p[src])
    missing = [k for k in keys if k not in sd and "position_ids" not in k]
    assert not missing, missing
    m.load_state_dict(sd, strict=False)
    return m


def _ids(B, vocab, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(2, vocab, size=(B, clip_ref.SEQ))
    ids[:, 0] = 0
    ids[:, -5:] = 1  # eos / padding tail, as a tokenizer pads to 77
    return ids


def _compare(p, ids, heads, **cfg):
    m = _hf_model(p, heads=heads, **cfg)
    with torch.inference_mode():
        ref = m(input_ids=torch.as_tensor(ids)).last_hidden_state.numpy()
        got = clip_ref.encode(p, ids, heads=heads).numpy()
    return np.abs(got - ref).max(), np.abs(ref).max()


SMALL = dict(vocab=1000, hidden=64, layers=3, ffn=256)


@pytest.mark.parametrize("mode", ["baseline", "affine"])
def test_small_config_matches_transformers(mode):
    p = clip_ref.generate(7, mode, **SMALL)
    err, mag = _compare(p, _ids(2, 1000, 1), heads=4, **SMALL)
    assert err < 2e-5 * max(mag, 1.0), (err, mag)


def test_full_config_matches_transformers():
    """SD1.5's text encoder shape: vocab 49408, 12 layers of 768, 12 heads, FFN 3072."""
    p = clip_ref.generate(11, "affine")
    err, mag = _compare(p, _ids(1, clip_ref.VOCAB, 2), heads=clip_ref.HEADS, vocab=clip_ref.VOCAB,
                        hidden=clip_ref.HIDDEN, layers=clip_ref.LAYERS, ffn=clip_ref.FFN)
    assert err < 5e-5 * max(mag, 1.0), (err, mag)


def test_planted_mistakes_fail(monkeypatch):
    p = clip_ref.generate(7, "affine", **SMALL)
    ids = _ids(2, 1000, 3)

    def no_mask(q, k, v, heads):
        B, S, C = q.shape
        d = C // heads
        qq = q.view(B, S, heads, d).transpose(1, 2) * d ** -0.5
        kk = k.view(B, S, heads, d).transpose(1, 2)
        vv = v.view(B, S, heads, d).transpose(1, 2)
        o = torch.softmax(qq @ kk.transpose(-1, -2), -1) @ vv
        return o.transpose(1, 2).reshape(B, S, C)

    for name, val in (("causal_attention", no_mask), ("quick_gelu", torch.nn.functional.gelu)):
        with monkeypatch.context() as mp:
            mp.setattr(clip_ref, name, val)
            err, mag = _compare(p, ids, heads=4, **SMALL)
            assert err > 1e-3 * mag, name

    # post-LayerNorm (LN applied after each residual add) instead of pre-LayerNorm
    def post_ln_encode(p_, ids_, heads=4):
        pt = {k: torch.as_tensor(np.asarray(v)) for k, v in p_.items()}
        idt = torch.as_tensor(ids_)
        pre = clip_ref.PREFIX
        x = pt[pre + "embeddings.token_embedding.weight"][idt] + pt[pre + "embeddings.position_embedding.weight"][None]
        C = x.shape[-1]
        for i in range(SMALL["layers"]):
            pf = f"{pre}encoder.layers.{i}"
            lin = lambda n, t: torch.nn.functional.linear(t, pt[f"{pf}.{n}.weight"], pt[f"{pf}.{n}.bias"])
            a = clip_ref.causal_attention(lin("self_attn.q_proj", x), lin("self_attn.k_proj", x),
                                          lin("self_attn.v_proj", x), heads)
            x = torch.nn.functional.layer_norm(x + lin("self_attn.out_proj", a), (C,), pt[pf + ".layer_norm1.weight"],
                                               pt[pf + ".layer_norm1.bias"], clip_ref.EPS)
            x = torch.nn.functional.layer_norm(x + lin("mlp.fc2", clip_ref.quick_gelu(lin("mlp.fc1", x))), (C,),
                                               pt[pf + ".layer_norm2.weight"], pt[pf + ".layer_norm2.bias"],
                                               clip_ref.EPS)
        return torch.nn.functional.layer_norm(x, (C,), pt[pre + "final_layer_norm.weight"],
                                              pt[pre + "final_layer_norm.bias"], clip_ref.EPS)

    with monkeypatch.context() as mp:
        mp.setattr(clip_ref, "encode", post_ln_encode)
        err, mag = _compare(p, ids, heads=4, **SMALL)
        assert err > 1e-3 * mag, "post-LN"


def test_inventory():
    """123.06 M parameters in 196 tensors (SD1.5's text encoder)."""
    ps = clip_ref.param_specs()
    assert len(ps) == 2 + 16 * 12 + 2
    assert sum(p.numel for p in ps) == 123_060_480
