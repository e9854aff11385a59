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
    d, V, f, L = cfg.d_model, cfg.vocab, cfg.d_ff, cfg.n_layers
    kvd = cfg.n_kv_heads * (d // cfg.n_heads)
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


# ---- the generic reader (rkv_st_*): any named-parameter model -----------------

def test_reader_lists_entries_like_the_safetensors_package(tmp_path):
    import torch
    from safetensors.torch import save_file as save_torch
    t = {"a.weight": torch.randn(3, 5), "b.half": torch.randn(7).half(),
         "c.bf16": torch.randn(2, 2, 2).bfloat16(), "d.ids": torch.arange(6, dtype=torch.int64),
         "e.scalar": torch.tensor(1.5)}
    path = tmp_path / "mixed.safetensors"
    save_torch(t, str(path), metadata={"k": "v"})
    want = {"a.weight": ("F32", (3, 5)), "b.half": ("F16", (7,)), "c.bf16": ("BF16", (2, 2, 2)),
            "d.ids": ("I64", (6,)), "e.scalar": ("F32", ())}
    with model.SafetensorsFile(path) as f:
        assert f.entries() == want


def test_generic_load_is_strict_and_exact(tmp_path):
    rng = np.random.default_rng(0)
    t = {"model.layers.0.self_attn.q_proj.weight": rng.standard_normal((8, 16), np.float32),
         "model.layers.0.self_attn.k_proj.weight": rng.standard_normal((4, 16), np.float32),
         "model.norm.weight": rng.standard_normal(16, np.float32)}
    path = tmp_path / "layer.safetensors"
    save_file(t, str(path))
    with model.SafetensorsFile(path) as f:
        dst = {k: np.empty_like(v) for k, v in t.items()}
        f.load(dst)
        for k in t:
            assert np.array_equal(dst[k], t[k]), k
        with pytest.raises(RkvError, match="unexpected extra keys: model.norm.weight"):
            f.load({k: np.empty_like(v) for k, v in t.items() if k != "model.norm.weight"})
        with pytest.raises(RkvError, match="missing keys: lm_head.weight"):
            f.load({**{k: np.empty_like(v) for k, v in t.items()},
                    "lm_head.weight": np.empty(3, np.float32)})
        bad = {k: np.empty_like(v) for k, v in t.items()}
        bad["model.norm.weight"] = np.empty((4, 4), np.float32)
        with pytest.raises(RkvError, match=r"shape mismatch for 'model.norm.weight': "
                                           r"expected \[4, 4\], got \[16\]"):
            f.load(bad)


def test_reader_rejects_malformed_headers(tmp_path):
    def write(header: bytes, body: bytes = b"", name="m.safetensors"):
        p = tmp_path / name
        p.write_bytes(len(header).to_bytes(8, "little") + header + body)
        return p
    cases = [
        (b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}', b"\0" * 8, "bad data_offsets"),
        (b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', b"\0" * 4, "bad data_offsets"),
        (b'{"a":{"dtype":"F32","shape":[-2],"data_offsets":[0,8]}}', b"\0" * 8, "bad shape"),
        (b'{"a":{"dtype":"F32","shape":[2.5],"data_offsets":[0,8]}}', b"\0" * 8, "bad shape"),
        (b'{"a":{"dtype":"F32","shape":[2]}}', b"\0" * 8, "malformed entry"),
        (b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},'
         b'"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', b"\0" * 8, "duplicate entry"),
        (b'[1,2]', b"", "not a JSON object"),
        # the data section is the tensors' ranges end to end, as the
        # safetensors package's validation requires (crates/io/src/lib.rs:150
        # loads through SafeTensors::deserialize)
        (b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},'
         b'"b":{"dtype":"F32","shape":[2],"data_offsets":[4,12]}}', b"\0" * 12, "overlaps"),
        (b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},'
         b'"b":{"dtype":"F32","shape":[2],"data_offsets":[12,20]}}', b"\0" * 20, "leaves a gap"),
        (b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[4,12]}}', b"\0" * 12, "leaves a gap"),
        (b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', b"\0" * 12,
         "4 data bytes past the last tensor"),
        (b'{}', b"\0", "1 data bytes past the last tensor"),
        (b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}x', b"\0" * 8,
         "trailing characters"),
        (b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}} {}', b"\0" * 8,
         "trailing characters"),
    ]
    for i, (h, body, msg) in enumerate(cases):
        with pytest.raises(RkvError, match=msg):
            model.SafetensorsFile(write(h, body, f"m{i}.safetensors"))
    short = tmp_path / "short.safetensors"
    short.write_bytes(b"\x01\x02")
    with pytest.raises(RkvError, match="shorter than 8 bytes"):
        model.SafetensorsFile(short)


def test_reader_accepts_space_padding_and_out_of_order_entries(tmp_path):
    """Spaces after the header object (the writer's 8-byte padding) are
    allowed, and header order need not be offset order: only the byte ranges
    must tile the data section."""
    h = (b'{"b":{"dtype":"F32","shape":[1],"data_offsets":[8,12]},'
         b'"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}   ')
    body = np.float32([1.0, 2.0, 3.0]).tobytes()
    p = tmp_path / "ok.safetensors"
    p.write_bytes(len(h).to_bytes(8, "little") + h + body)
    with model.SafetensorsFile(p) as f:
        assert set(f.entries()) == {"a", "b"}
        out = {"a": np.empty(2, np.float32), "b": np.empty(1, np.float32)}
        f.load(out)
    assert out["a"].tolist() == [1.0, 2.0] and out["b"].tolist() == [3.0]
