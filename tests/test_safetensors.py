"""Decoder parameters in safetensors files (host code, CPU tests): the writer
and the strict loader against the independent `safetensors` package, and the
reference's strictness rules (crates/runtime/src/model_io.rs:36-105)."""
import numpy as np
import pytest
from safetensors.numpy import load_file, save_file

from rustral_amd import model
from rustral_amd._lib import RkvError

CFG = dict(vocab=50, d_model=64, n_heads=4, n_kv_heads=2, d_ff=96, n_layers=2, max_seq=32)


def named(cfg, params):
    """The name -> array view of a packed parameter array, from the names and
    shapes the header documents (an independent walk of the layout)."""
    c = dict(model.CONFIG0)
    c.update(CFG)
    d, V, f, L = c["d_model"], c["vocab"], c["d_ff"], c["n_layers"]
    kvd = c["n_kv_heads"] * (d // c["n_heads"])
    order = [("token_embedding.weight", (V, d))]
    for i in range(L):
        p = f"layers.{i}."
        order += [(p + "norm1.weight", (d,)), (p + "norm1.bias", (d,)),
                  (p + "self_attn.q_proj.weight", (d, d)), (p + "self_attn.q_proj.bias", (d,)),
                  (p + "self_attn.k_proj.weight", (kvd, d)), (p + "self_attn.k_proj.bias", (kvd,)),
                  (p + "self_attn.v_proj.weight", (kvd, d)), (p + "self_attn.v_proj.bias", (kvd,)),
                  (p + "self_attn.out_proj.weight", (d, d)), (p + "self_attn.out_proj.bias", (d,)),
                  (p + "norm2.weight", (d,)), (p + "norm2.bias", (d,)),
                  (p + "ff_linear1.weight", (f, d)), (p + "ff_linear1.bias", (f,)),
                  (p + "ff_linear2.weight", (d, f)), (p + "ff_linear2.bias", (d,))]
    order += [("final_norm.weight", (d,)), ("final_norm.bias", (d,)), ("lm_head.weight", (V, d))]
    out, o = {}, 0
    for name, shape in order:
        n = int(np.prod(shape))
        out[name] = params[o:o + n].reshape(shape)
        o += n
    assert o == params.size
    return out


@pytest.fixture
def cfg():
    return model.config(**CFG)


def test_writer_output_reads_back_with_the_safetensors_package(cfg, tmp_path):
    params = model.init_params(cfg, seed=3, std=0.5)
    path = tmp_path / "dec.safetensors"
    model.save_safetensors(cfg, params, path)
    got = load_file(str(path))
    want = named(cfg, params)
    assert set(got) == set(want)
    for k in want:
        assert got[k].dtype == np.float32 and got[k].shape == want[k].shape
        assert np.array_equal(got[k], want[k]), k


def test_loader_reads_the_safetensors_package_output(cfg, tmp_path):
    params = model.init_params(cfg, seed=4, std=0.5)
    path = tmp_path / "dec.safetensors"
    tensors = {k: np.ascontiguousarray(v) for k, v in named(cfg, params).items()}
    save_file(tensors, str(path), metadata={"rustral.parameter_ids": "{}"})
    assert np.array_equal(model.load_safetensors(cfg, path), params)
    # round trip through the library's own writer
    path2 = tmp_path / "dec2.safetensors"
    model.save_safetensors(cfg, params, path2)
    assert np.array_equal(model.load_safetensors(cfg, path2), params)


def _write_modified(cfg, tmp_path, edit):
    params = model.init_params(cfg, seed=5)
    tensors = {k: np.ascontiguousarray(v) for k, v in named(cfg, params).items()}
    edit(tensors)
    path = tmp_path / "bad.safetensors"
    save_file(tensors, str(path))
    return path


@pytest.mark.parametrize("edit,message", [
    (lambda t: t.pop("layers.1.norm2.bias"), "missing keys: layers.1.norm2.bias"),
    (lambda t: t.update({"extra.weight": np.zeros(3, np.float32)}),
     "unexpected extra keys: extra.weight"),
    (lambda t: t.update({"lm_head.weight": np.zeros((64, 50), np.float32)}),
     "shape mismatch for 'lm_head.weight': expected [50, 64], got [64, 50]"),
    (lambda t: t.update({"final_norm.bias": np.zeros(64, np.float16)}),
     "dtype mismatch for 'final_norm.bias': expected F32, got F16"),
])
def test_loader_is_strict_like_load_model(cfg, tmp_path, edit, message):
    path = _write_modified(cfg, tmp_path, edit)
    with pytest.raises(RkvError) as e:
        model.load_safetensors(cfg, path)
    assert message in str(e.value)


def test_loader_rejects_truncated_and_missing_files(cfg, tmp_path):
    good = tmp_path / "good.safetensors"
    model.save_safetensors(cfg, model.init_params(cfg, seed=6), good)
    data = good.read_bytes()
    cut = tmp_path / "cut.safetensors"
    cut.write_bytes(data[:-100])
    with pytest.raises(RkvError, match="bad data_offsets"):
        model.load_safetensors(cfg, cut)
    junk = tmp_path / "junk.safetensors"
    junk.write_bytes(b"\x05\x00\x00\x00\x00\x00\x00\x00{bad}")
    with pytest.raises(RkvError, match="not a JSON object"):
        model.load_safetensors(cfg, junk)
    with pytest.raises(RkvError, match="cannot open"):
        model.load_safetensors(cfg, tmp_path / "absent.safetensors")
