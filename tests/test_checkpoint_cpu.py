"""CPU tests of the safetensors checkpoint reader (gptoss_checkpoint_*):
the index and bytes match what the `safetensors` package itself wrote and
reads back, malformed files fail with a status code instead of aborting
(the reference aborts, weight_loader.cu:493-531), and the MoE layer loader
resolves GPT-OSS tensor names and checks shapes and dtypes on the host before
it touches a device (weight_loader.cu:818-895, 1083-1165)."""
import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

import ckpt_data
import moe_data


@pytest.fixture(scope="module")
def g():
    import gptoss_moe
    return gptoss_moe


def _mixed_tensors():
    rng = np.random.default_rng(5)
    return {
        "model.embed_tokens.weight": torch.from_numpy(rng.normal(size=(7, 5)).astype(np.float32)).to(torch.bfloat16),
        "a.f32": torch.from_numpy(rng.normal(size=(3, 4, 2)).astype(np.float32)),
        "a.f16": torch.from_numpy(rng.normal(size=(9,)).astype(np.float16)),
        "a.u8": torch.from_numpy(rng.integers(0, 256, (4, 6, 16), dtype=np.uint8)),
        "a.i64": torch.arange(-3, 5, dtype=torch.int64),
        "a.bool": torch.tensor([True, False, True]),
        "a.scalar": torch.tensor(2.5, dtype=torch.float32),
        "a.empty": torch.zeros((0, 3), dtype=torch.float32),
        "b.ünïcode name": torch.ones((2,), dtype=torch.int32),
    }


def test_index_and_bytes_match_safetensors(g, tmp_path):
    tensors = _mixed_tensors()
    paths = ckpt_data.write_shards(str(tmp_path), tensors, n_shards=3, metadata={"format": "pt", "x": "{\"y\": [1]}"})
    with g.Checkpoint(str(tmp_path)) as ck:
        assert sorted(ck.names()) == sorted(tensors)
        assert len(ck) == len(tensors)
        for i, p in enumerate(sorted(paths)):
            with safe_open(p, framework="pt") as f:
                for n in f.keys():
                    ref = f.get_tensor(n)
                    inf = ck.info(n)
                    assert inf["shape"] == tuple(ref.shape), n
                    assert inf["shard"] == i
                    want = {torch.bfloat16: "BF16", torch.float32: "F32", torch.float16: "F16", torch.uint8: "U8",
                            torch.int64: "I64", torch.bool: "BOOL", torch.int32: "I32"}[ref.dtype]
                    assert inf["dtype"] == want
                    raw = ref.reshape(-1).contiguous().view(torch.uint8).numpy().tobytes() if ref.numel() else b""
                    assert inf["nbytes"] == len(raw)
                    got = ck.numpy(n)
                    assert got.tobytes() == raw, n
                    assert got.shape == tuple(ref.shape)
        assert ck.info("not.there") is None


def test_single_file_and_later_shard_wins(g, tmp_path):
    a = {"w": torch.zeros(4, dtype=torch.float32), "only_a": torch.ones(2, dtype=torch.float32)}
    b = {"w": torch.full((4,), 7.0, dtype=torch.float32)}
    save_file(a, str(tmp_path / "model-00001.safetensors"))
    save_file(b, str(tmp_path / "model-00002.safetensors"))
    (tmp_path / "notes.txt").write_text("not a shard")
    with g.Checkpoint(str(tmp_path)) as ck:
        assert np.array_equal(ck.numpy("w"), np.full(4, 7.0, np.float32))  # name order: 00002 last
        assert ck.info("w")["shard"] == 1
    with g.Checkpoint(str(tmp_path / "model-00001.safetensors")) as ck:
        assert sorted(ck.names()) == ["only_a", "w"]
        assert np.array_equal(ck.numpy("w"), np.zeros(4, np.float32))


def _raw_file(path, header, data=b"", hlen=None):
    hb = header if isinstance(header, bytes) else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb) if hlen is None else hlen))
        f.write(hb)
        f.write(data)


def test_hand_written_headers(g, tmp_path):
    # padding spaces after the object, escapes in names, unknown keys and a
    # nested __metadata__ are all accepted
    hdr = (b'{"__metadata__": {"k": "v"}, "a\\u00e9\\"b\\ud83d\\ude00": {"dtype": "U8", "shape": [2, 2],'
           b' "data_offsets": [0, 4], "extra": [1, {"z": null}]}}   ')
    p = tmp_path / "x.safetensors"
    _raw_file(p, hdr, bytes([1, 2, 3, 4]))
    with g.Checkpoint(str(p)) as ck:
        assert ck.names() == ['aé"b\U0001F600']
        assert ck.numpy('aé"b\U0001F600').tolist() == [[1, 2], [3, 4]]


@pytest.mark.parametrize("case", ["short", "hlen", "json", "trailing", "past_end", "size", "no_offsets",
                                  "neg_shape", "float_offset", "bad_utf8", "cut_utf8", "lone_surrogate", "nul"])
def test_malformed_files_fail_with_io(g, tmp_path, case):
    p = tmp_path / "bad.safetensors"
    ok_entry = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}
    if case == "short":
        p.write_bytes(b"\x01\x00")
    elif case == "hlen":
        _raw_file(p, {"t": ok_entry}, bytes(8), hlen=1 << 40)
    elif case == "json":
        _raw_file(p, b'{"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}', bytes(8))
    elif case == "trailing":
        _raw_file(p, b'{"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}} x', bytes(8))
    elif case == "past_end":
        _raw_file(p, {"t": ok_entry}, bytes(4))
    elif case == "size":
        _raw_file(p, {"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "no_offsets":
        _raw_file(p, {"t": {"dtype": "F32", "shape": [2]}}, bytes(8))
    elif case == "neg_shape":
        _raw_file(p, {"t": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "float_offset":
        _raw_file(p, b'{"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8.0]}}', bytes(8))
    elif case == "bad_utf8":   # a name that is not UTF-8 (JSON text must be)
        _raw_file(p, b'{"t\xd6x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}', bytes(8))
    elif case == "cut_utf8":   # a multi-byte sequence cut by the closing quote
        _raw_file(p, b'{"t\xe2\x82": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}', bytes(8))
    elif case == "lone_surrogate":
        _raw_file(p, b'{"t\\ud83d": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}', bytes(8))
    elif case == "nul":
        _raw_file(p, b'{"t\\u0000x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}', bytes(8))
    with pytest.raises(g.GptossError) as e:
        g.Checkpoint(str(p))
    assert e.value.code == g.GPTOSS_ERR_IO, str(e.value)
    assert "bad.safetensors" in str(e.value)


def test_mutated_headers_fail_cleanly(g, tmp_path):
    """Seeded mutations of a valid header (byte flips, inserted and deleted
    bytes, truncations, a wrong length prefix): every open either succeeds
    with tensors whose byte ranges lie inside the file or fails with a status
    code.  Under tests/sanitize (ASan + UBSan) this is the parser's fuzz pass."""
    hdr = json.dumps({"__metadata__": {"format": "pt"},
                      "a.w": {"dtype": "BF16", "shape": [3, 4], "data_offsets": [0, 24]},
                      "b\u00e9": {"dtype": "U8", "shape": [8], "data_offsets": [24, 32]},
                      "c": {"dtype": "F32", "shape": [], "data_offsets": [32, 36]}}).encode()
    data = bytes(range(36))
    rng = np.random.default_rng(11)
    p = tmp_path / "m.safetensors"
    n_ok = 0
    for it in range(400):
        h = bytearray(hdr)
        for _ in range(int(rng.integers(1, 4))):
            op = int(rng.integers(0, 4))
            i = int(rng.integers(0, len(h))) if h else 0
            if op == 0 and h:
                h[i] = int(rng.integers(0, 256))
            elif op == 1:
                h[i:i] = bytes([int(rng.choice(list(b'{}[]",:0-9e.\\u ')))])
            elif op == 2 and h:
                del h[i]
            else:
                h = h[:i]
        hlen = len(h) + int(rng.integers(-3, 4)) if it % 7 == 0 else len(h)
        p.write_bytes(struct.pack("<Q", max(hlen, 0)) + bytes(h) + data)
        try:
            ck = g.Checkpoint(str(p))
        except g.GptossError as e:
            assert e.code in (g.GPTOSS_ERR_IO, g.GPTOSS_ERR_INVALID), str(e)
            continue
        with ck:
            for n in ck.names():
                inf = ck.info(n)
                assert inf["nbytes"] <= len(data)
                ck.numpy(n)
            n_ok += 1
    assert 0 < n_ok < 400


def test_missing_paths(g, tmp_path):
    with pytest.raises(g.GptossError) as e:
        g.Checkpoint(str(tmp_path / "nope"))
    assert e.value.code == g.GPTOSS_ERR_NOT_FOUND
    with pytest.raises(g.GptossError) as e:
        g.Checkpoint(str(tmp_path))  # a directory without shards
    assert e.value.code == g.GPTOSS_ERR_NOT_FOUND
    assert g.lib.gptoss_checkpoint_open(None, None) == g.GPTOSS_ERR_INVALID


# ---- the MoE layer loader's host-side checks --------------------------------
E, H, I = 4, 64, 64


def _layer_dir(tmp_path, fmt="packed", mutate=None, **kw):
    w = moe_data.make_layer(3, E, H, I, bias="random")
    t = ckpt_data.layer_tensors(0, w, E, H, I, fmt=fmt, norm_w=moe_data.bf16(np.ones(H)), **kw)
    if mutate:
        mutate(t)
    d = tmp_path / "ck"
    ckpt_data.write_shards(str(d), t, n_shards=2)
    return str(d)


def _init(g, path, layer=0, e=E):
    cfg = g.default_config(e, 8)
    cfg.hidden_size, cfg.intermediate_size = H, I
    L = g.MoELayer()
    with g.Checkpoint(path) as ck:
        try:
            L.init_from_checkpoint(cfg, 0, ck, layer)
        finally:
            L.destroy()


def _expect(g, path, code, text, **kw):
    with pytest.raises(g.GptossError) as e:
        _init(g, path, **kw)
    assert e.value.code == code, str(e.value)
    assert text in str(e.value), str(e.value)


P = "model.layers.0."


def test_layer_loader_resolution_errors(g, tmp_path):
    _expect(g, _layer_dir(tmp_path), g.GPTOSS_ERR_NOT_FOUND, "model.layers.1.mlp.gate.weight", layer=1)
    _expect(g, _layer_dir(tmp_path), g.GPTOSS_ERR_INVALID, "layer_index=-1", layer=-1)
    # the checkpoint has 4 experts, the config asks for 8
    _expect(g, _layer_dir(tmp_path), g.GPTOSS_ERR_INVALID, "router.weight", e=8)


@pytest.mark.parametrize("what", ["router_shape", "router_dtype", "blocks_shape", "scales_missing", "down_missing",
                                  "bias_shape", "expert_missing", "expert_scale_missing", "expert_rows"])
def test_layer_loader_shape_and_name_errors(g, tmp_path, what):
    fmt = "per_expert" if what.startswith("expert") else "packed"

    def mutate(t):
        if what == "router_shape":
            t[P + "mlp.router.weight"] = t[P + "mlp.router.weight"].reshape(H, E).contiguous()
        elif what == "router_dtype":
            t[P + "mlp.router.weight"] = torch.zeros((E, H), dtype=torch.int32)
        elif what == "blocks_shape":
            t[P + "mlp.experts.gate_up_proj_blocks"] = t[P + "mlp.experts.gate_up_proj_blocks"][:, :64].contiguous()
        elif what == "scales_missing":
            del t[P + "mlp.experts.down_proj_scales"]
        elif what == "down_missing":
            del t[P + "mlp.experts.down_proj_blocks"]
        elif what == "bias_shape":
            t[P + "mlp.experts.down_proj_bias"] = t[P + "mlp.experts.down_proj_bias"][:, :32].contiguous()
        elif what == "expert_missing":
            del t[P + "mlp.experts.2.mlp2.weight"]
        elif what == "expert_scale_missing":
            del t[P + "mlp.experts.3.mlp1.weight_scale"]
        elif what == "expert_rows":
            t[P + "mlp.experts.1.mlp1.weight"] = t[P + "mlp.experts.1.mlp1.weight"][:64].contiguous()

    code, text = {
        "router_shape": (g.GPTOSS_ERR_INVALID, "expected [4,64]"),
        "router_dtype": (g.GPTOSS_ERR_INVALID, "dtype I32"),
        "blocks_shape": (g.GPTOSS_ERR_INVALID, "gate_up_proj_blocks"),
        "scales_missing": (g.GPTOSS_ERR_NOT_FOUND, "down_proj_blocks' has no scales"),
        "down_missing": (g.GPTOSS_ERR_NOT_FOUND, "down_proj_blocks"),
        "bias_shape": (g.GPTOSS_ERR_INVALID, "down_proj_bias"),
        "expert_missing": (g.GPTOSS_ERR_NOT_FOUND, "expert 2"),
        "expert_scale_missing": (g.GPTOSS_ERR_NOT_FOUND, "expert 3"),
        "expert_rows": (g.GPTOSS_ERR_INVALID, "experts.1.mlp1.weight"),
    }[what]
    _expect(g, _layer_dir(tmp_path, fmt=fmt, mutate=mutate), code, text)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the host-side pass on a host without a GPU")
@pytest.mark.parametrize("fmt,kw", [("packed", {}), ("per_expert", {}),
                                    ("per_expert", {"expert_names": ("gate_up_proj", "down_proj")}),
                                    ("packed", {"router_name": "gate"})])
def test_layer_loader_accepts_valid_layouts_on_host(g, tmp_path, fmt, kw):
    """Every host-side check passes: the call gets as far as selecting the
    device, which fails here for want of one."""
    with pytest.raises(g.GptossError) as e:
        _init(g, _layer_dir(tmp_path, fmt=fmt, **kw))
    assert e.value.code == g.GPTOSS_ERR_HIP, str(e.value)


def test_stack_and_engine_host_errors(g, tmp_path):
    """Argument errors of the stack and the engine surface, caught before any
    device work."""
    import ctypes
    out = ctypes.c_void_p()
    assert g.lib.gptoss_moe_stack_create_from_layers(None, 1, ctypes.byref(out)) == g.GPTOSS_ERR_INVALID
    L = g.MoELayer()  # created, never initialised
    arr = (ctypes.c_void_p * 1)(L._h)
    assert g.lib.gptoss_moe_stack_create_from_layers(arr, 0, ctypes.byref(out)) == g.GPTOSS_ERR_INVALID
    assert g.lib.gptoss_moe_stack_create_from_layers(arr, 1, ctypes.byref(out)) == g.GPTOSS_ERR_STATE
    assert b"not initialised" in g.lib.gptoss_last_error()
    L.destroy()
    assert g.lib.gptoss_moe_stack_decode_step(None, 1, g._HOOK(), None, 1, None) == g.GPTOSS_ERR_INVALID
    cfg = g.default_config(4, 8)
    assert g.lib.gptoss_moe_stack_create(ctypes.byref(cfg), 0, None, 0, 1, ctypes.byref(out)) == g.GPTOSS_ERR_INVALID
    eng = g.MoEEngine()
    assert not eng.is_initialized and repr(eng) == "<gptoss_moe.MoEEngine initialized=False layers=0>"
    with pytest.raises(g.GptossError) as e:
        eng.init(str(tmp_path / "missing"))
    assert e.value.code == g.GPTOSS_ERR_NOT_FOUND
    with pytest.raises(g.GptossError):
        eng.stack
    assert (g.ModelConfig.num_layers, g.ModelConfig.num_experts, g.ModelConfig.num_active_experts) == (36, 128, 4)


def test_checkpoint_moe_shape_detection(g, tmp_path):
    for fmt, kw in (("packed", {}), ("per_expert", {"expert_names": ("gate_up_proj", "down_proj")})):
        d = tmp_path / fmt
        w = moe_data.make_layer(3, E, H, I)
        t = {}
        for l in range(3):
            t.update(ckpt_data.layer_tensors(l, w, E, H, I, fmt=fmt, **kw))
        ckpt_data.write_shards(str(d), t, n_shards=2)
        with g.Checkpoint(str(d)) as ck:
            assert ck.moe_shape(0) == (E, H, I)
            assert ck.num_moe_layers() == 3
