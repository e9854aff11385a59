"""Safetensors weights straight into device buffers (GPU): the reference's
strict load_model (crates/runtime/src/model_io.rs:36-105) feeding the device
path.

* the decoder's weights written by the independent `safetensors`
  package, loaded with rkv_decoder_create_from_safetensors into device
  memory; the 64 greedy tokens equal the CPU oracle's.
* one Llama-3-8B attention layer (d_model 4096, 32 query heads, 8 KV heads,
  head_dim 128): q/k/v/o projection weights loaded with rkv_st_load into
  device tensors feed rkv_qkv_append (bf16 pools) and the output projection;
  bit-equal to the oracle's linear + append.
"""
import numpy as np
import pytest
from safetensors.numpy import save_file

import oracle
from rustral_amd import model
from rustral_amd._lib import RkvError
from tests.gpu_util import say
from tests.test_safetensors import named

pytestmark = pytest.mark.gpu


def _named0(cfg, params):
    return {k: np.ascontiguousarray(v) for k, v in named(cfg, params).items()}


def test_config0_decoder_from_safetensors_tokens_equal_oracle(dev, tmp_path):
    say("decoder configs[0] from a safetensors file")
    cfg = model.config()
    params = model.init_params(cfg, seed=0, std=0.02)
    path = tmp_path / "config0.safetensors"
    save_file(_named0(cfg, params), str(path), metadata={"format": "pt"})
    prompt = np.random.default_rng(0).integers(0, 1000, 32).astype(np.int32)
    dec = model.Decoder(cfg, path=path)
    toks = dec.generate(prompt, 64)
    want = oracle.decoder_generate(oracle.decoder_config(), params, prompt, 64)
    assert toks.tolist() == want.tolist()
    # replace the weights of the live decoder from another file
    params2 = model.init_params(cfg, seed=7, std=0.02)
    path2 = tmp_path / "config0_seed7.safetensors"
    save_file(_named0(cfg, params2), str(path2))
    dec.load_safetensors(path2)
    want2 = oracle.decoder_generate(oracle.decoder_config(), params2, prompt, 64)
    assert dec.generate(prompt, 64).tolist() == want2.tolist()
    # a strictness failure leaves the decoder's parameters as they were
    bad = _named0(cfg, params)
    bad.pop("lm_head.weight")
    path3 = tmp_path / "missing.safetensors"
    save_file(bad, str(path3))
    with pytest.raises(RkvError, match="missing keys: lm_head.weight"):
        dec.load_safetensors(path3)
    assert dec.generate(prompt, 64).tolist() == want2.tolist()
    with pytest.raises(RkvError, match="missing keys: lm_head.weight"):
        model.Decoder(cfg, path=path3)


def test_llama3_8b_layer_projections_from_safetensors_feed_qkv_append(dev, tmp_path):
    import torch
    say("Llama-3-8B layer q/k/v/o from safetensors -> qkv_append + o_proj")
    d, hq, hkv, hd = 4096, 32, 8, 128
    rng = np.random.default_rng(8)
    pre = "model.layers.0.self_attn."
    w = {pre + "q_proj.weight": (rng.standard_normal((hq * hd, d)) * 0.02).astype(np.float32),
         pre + "k_proj.weight": (rng.standard_normal((hkv * hd, d)) * 0.02).astype(np.float32),
         pre + "v_proj.weight": (rng.standard_normal((hkv * hd, d)) * 0.02).astype(np.float32),
         pre + "o_proj.weight": (rng.standard_normal((d, hq * hd)) * 0.02).astype(np.float32)}
    path = tmp_path / "llama_layer0.safetensors"
    save_file(w, str(path))
    gw = {k: torch.empty(v.shape, dtype=torch.float32, device=dev) for k, v in w.items()}
    with model.SafetensorsFile(path) as f:
        f.load(gw)
    torch.cuda.synchronize()
    for k in w:
        assert np.array_equal(gw[k].cpu().numpy(), w[k]), k
    n, nb, bs = 5, 4, 16
    x = (rng.standard_normal((n, d)) * 1.5).astype(np.float32)
    slots = rng.permutation(nb * bs)[:n].astype(np.int64)
    kp = oracle.bf16_from_f32(rng.standard_normal((nb, hkv, bs, hd)).astype(np.float32))
    vp = oracle.bf16_from_f32(rng.standard_normal((nb, hkv, bs, hd)).astype(np.float32))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    gk = torch.from_numpy(kp.view(np.int16)).to(dev).view(torch.bfloat16)
    gv = torch.from_numpy(vp.view(np.int16)).to(dev).view(torch.bfloat16)
    q = model.qkv_append(t(x), gw[pre + "q_proj.weight"], gw[pre + "k_proj.weight"],
                         gw[pre + "v_proj.weight"], gk, gv, t(slots))
    o = model.linear(q, gw[pre + "o_proj.weight"])
    torch.cuda.synchronize()
    want_q = oracle.linear(x, w[pre + "q_proj.weight"])
    want_k, want_v = kp.copy(), vp.copy()
    oracle.append(want_k, want_v, oracle.linear(x, w[pre + "k_proj.weight"]).reshape(n, hkv, hd),
                  oracle.linear(x, w[pre + "v_proj.weight"]).reshape(n, hkv, hd), slots)
    assert np.array_equal(q.cpu().numpy(), want_q)
    assert np.array_equal(gk.view(torch.int16).cpu().numpy().view(np.uint16), want_k)
    assert np.array_equal(gv.view(torch.int16).cpu().numpy().view(np.uint16), want_v)
    assert np.array_equal(o.cpu().numpy(), oracle.linear(want_q, w[pre + "o_proj.weight"]))
