"""GGUF parsing, KV sizing and the `ts5 check` file format of the C-ABI
library, on the CPU (no GPU call is made here).

Pins:
* kv_bytes_per_token against what the cache layout fixes for cfg2 (32 layers
  x 8 KV heads x 128 values x K and V: 69,632 B in q8, a byte per value and
  an f16 scale per 32, engine/src/vk_backend.cpp:1374-1376) and fit_context /
  f16_reaches on their boundary cases (engine/src/vk_backend.cpp:1395-1402);
* the GGUF reader against files written by tests/golden/gguf_writer.py
  (hyperparameters as engine/src/model.cpp:13-68 derives them, including the
  qwen2 training-context clamp);
* the .ts5ref reader and writer against the files ts5's own run_check saved
  (tests/golden/check.npz, made by make_golden.py from engine/src/checks.cpp):
  the library reads the reference's file back as the oracle's logits for the
  check's test tokens, bit for bit, and writes a byte-identical file."""
import os

import numpy as np
import pytest

import gguf_writer
import make_golden
import oracle
from tokenstation5_amd import synth, ts5hip

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_kv_sizing():
    hp = synth.LLAMA_8B
    assert ts5hip.kv_bytes_per_token(hp, ts5hip.KV_Q8) == 69632
    assert ts5hip.kv_bytes_per_token(hp, ts5hip.KV_F16) == 131072
    assert ts5hip.kv_bytes_per_token(hp, ts5hip.KV_F32) == 262144
    gib = 1 << 30
    # What is left after `used` and 1 GiB, in whole 1024-token steps, at most cap.
    assert ts5hip.fit_context(10 * gib, 2 * gib, 131072, 1 << 20) == 57344
    assert ts5hip.fit_context(10 * gib, 2 * gib, 131072, 8192) == 8192
    assert ts5hip.fit_context(10 * gib, 2 * gib, 131072, 5000) == 4096
    assert ts5hip.fit_context(3 * gib, 2 * gib, 131072, 8192) == 0      # nothing past the reserve
    assert ts5hip.fit_context(2 * gib + 1023 * 131072, gib, 131072, 8192) == 0  # not even 1024 tokens
    assert ts5hip.fit_context(10 * gib, 2 * gib, 0, 8192) == 0
    assert ts5hip.f16_reaches(8192, 8192) and ts5hip.f16_reaches(8192, 8500)
    assert not ts5hip.f16_reaches(7168, 8192) and not ts5hip.f16_reaches(4096, 512)


@pytest.mark.parametrize("hp", [synth.TINY_LLAMA, synth.TINY_DRAFT, synth.TINY_GEMMA3])
def test_gguf_hparams(tmp_path, hp):
    path = str(tmp_path / "m.gguf")
    tensors = synth.model_tensors(hp, 3)
    gguf_writer.write(path, gguf_writer.model_kv(hp), tensors)
    got, train, fixed = ts5hip.gguf_hparams(path)
    want = ts5hip.hparams(hp)
    for f, _ in ts5hip.HParams._fields_:
        assert got[f] == pytest.approx(getattr(want, f)), f
    # qwen2 files declaring more than 32768 without RoPE-scaling keys keep 32768.
    assert train == 32768
    assert fixed > sum(v[3].nbytes for v in tensors.values())


def test_gguf_errors(tmp_path):
    bad = tmp_path / "x.gguf"
    bad.write_bytes(b"NOPE" + bytes(64))
    with pytest.raises(ts5hip.Ts5HipError):
        ts5hip.gguf_hparams(str(bad))
    # A gemma3 file without its layers' norms after attention and the FFN (model.cpp:114-116).
    hp = dict(synth.TINY_LLAMA, arch="gemma3")
    path = str(tmp_path / "g.gguf")
    gguf_writer.write(path, gguf_writer.model_kv(hp), synth.model_tensors(synth.TINY_LLAMA, 3))
    with pytest.raises(ts5hip.Ts5HipError, match="post_attention_norm"):
        ts5hip.gguf_hparams(path)
    hp = dict(synth.TINY_LLAMA, arch="mamba")
    gguf_writer.write(path, gguf_writer.model_kv(hp), synth.model_tensors(synth.TINY_LLAMA, 3))
    with pytest.raises(ts5hip.Ts5HipError, match="mamba"):
        ts5hip.gguf_hparams(path)
    trunc = str(tmp_path / "t.gguf")
    gguf_writer.write(trunc, gguf_writer.model_kv(synth.TINY_LLAMA), synth.model_tensors(synth.TINY_LLAMA, 3))
    with open(trunc, "r+b") as f:
        f.truncate(os.path.getsize(trunc) // 2)  # tensors past the end of the file
    with pytest.raises(ts5hip.Ts5HipError):
        ts5hip.gguf_hparams(trunc)


def test_gemma3_hparams(tmp_path, monkeypatch):
    """What the loader adds for gemma3 files (engine/src/model.cpp:44-63):
    sqrt(n_embd) embedding scale, GELU, a window on five layers of six with
    RoPE base 10000, the 27B's query scale 1/sqrt(n_embd / n_head) at 62
    layers, and TS5_SWA_WINDOW replacing the file's window."""
    hp = dict(synth.TINY_GEMMA3, n_layer=62, swa_window=1024)
    tensors = {k: v for k, v in synth.model_tensors(dict(synth.TINY_GEMMA3, n_layer=62), 3).items()
               if "norm" in k or k == "token_embd.weight"}  # hparams need no matrices
    path = str(tmp_path / "g62.gguf")
    gguf_writer.write(path, gguf_writer.model_kv(hp), tensors)
    got, train, _ = ts5hip.gguf_hparams(path)
    assert got["embd_scale"] == np.float32(np.sqrt(np.float32(512)))
    assert (got["gelu"], got["swa_window"], got["swa_pattern"], got["rope_base_swa"]) == (1, 1024, 6, 10000.0)
    assert got["attn_scale"] == np.float32(1) / np.sqrt(np.float32(512 // 4))  # not 1 / sqrt(head_dim 256)
    assert got["rope_neox"] == 1 and train == 32768
    monkeypatch.setenv("TS5_SWA_WINDOW", "16")
    assert ts5hip.gguf_hparams(path)[0]["swa_window"] == 16
    # Every layer keeps a full cache: K and V of all 62 layers per token.
    assert ts5hip.kv_bytes_per_token(hp, ts5hip.KV_F16) == 2 * 62 * 1 * 256 * 2


def check_model(tmp_path):
    """The GGUF make_golden.py handed to the reference's run_check, rewritten
    byte for byte (its sha256 is in check.npz)."""
    import hashlib
    path = str(tmp_path / "check.gguf")
    tensors = synth.model_tensors(make_golden.TINY_CHECK, make_golden.MODEL_SEED)
    gguf_writer.write(path, gguf_writer.model_kv(make_golden.TINY_CHECK), tensors)
    g = np.load(os.path.join(G, "check.npz"))
    assert hashlib.sha256(open(path, "rb").read()).digest() == bytes(g["gguf_sha"])
    return path, tensors, g


@pytest.mark.parametrize("kv", [ts5hip.KV_F16, ts5hip.KV_Q8])
def test_ref_file_matches_reference(tmp_path, kv):
    path, tensors, g = check_model(tmp_path)
    hp, n = make_golden.TINY_CHECK, make_golden.CHECK_N
    nv = hp["n_vocab"]
    ref_bytes = bytes(g[f"kv{kv}_file"])
    assert ts5hip.ref_path(path, kv) == path + (".ts5ref" if kv == ts5hip.KV_F16 else ".q8.ts5ref")
    with open(ts5hip.ref_path(path, kv), "wb") as f:
        f.write(ref_bytes)
    got = ts5hip.ref_load(path, n, nv, kv)
    # The oracle on the check's test tokens gives the saved logits bit for bit
    # (the check's tokens and the reference's CPU values, pinned together).
    toks = ts5hip.check_tokens(n, nv)
    m = oracle.Model(hp, tensors, n, kv)
    want = m.forward(toks, 0, all_logits=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # Fewer positions read the first ones; more than the file holds is refused.
    assert np.array_equal(ts5hip.ref_load(path, 5, nv, kv), got[:5])
    with pytest.raises(ts5hip.Ts5HipError):
        ts5hip.ref_load(path, n + 1, nv, kv)
    with pytest.raises(ts5hip.Ts5HipError):
        ts5hip.ref_load(path, n, nv, ts5hip.KV_F32)  # no file for that cache type
    # Writing: byte for byte the reference's file; a file with more positions is kept.
    os.remove(ts5hip.ref_path(path, kv))
    ts5hip.ref_save(path, kv, got)
    assert open(ts5hip.ref_path(path, kv), "rb").read() == ref_bytes
    ts5hip.ref_save(path, kv, got[:4])
    assert open(ts5hip.ref_path(path, kv), "rb").read() == ref_bytes
    # A different model file (same size, other bytes) no longer matches.
    with open(path, "r+b") as f:
        f.seek(100)
        f.write(b"\xff")
    with pytest.raises(ts5hip.Ts5HipError):
        ts5hip.ref_load(path, n, nv, kv)


def test_check_tokens():
    t = ts5hip.check_tokens(6, 128256)
    assert list(t) == [1000 + (i * 7919) % 127256 for i in range(6)]
    with pytest.raises(ts5hip.Ts5HipError):
        ts5hip.check_tokens(4, 1000)


def test_ref_save_replaces_another_models_file(tmp_path):
    """A saved file keeps its place only for the same model and cache type: a
    longer file of another model is replaced, and a file that is not a .ts5ref
    at all is refused on load."""
    path, tensors, g = check_model(tmp_path)
    hp, n = make_golden.TINY_CHECK, make_golden.CHECK_N
    kv = ts5hip.KV_Q8
    ref = ts5hip.ref_path(path, kv)
    with open(ref, "wb") as f:
        f.write(bytes(g[f"kv{kv}_file"]))
    got = ts5hip.ref_load(path, n, hp["n_vocab"], kv)
    other = str(tmp_path / "other.gguf")
    with open(path, "rb") as f:
        body = bytearray(f.read())
    body[100] ^= 0xFF
    with open(other, "wb") as f:
        f.write(body)
    # The other model's file holds more positions but is for other bytes.
    os.rename(ref, ts5hip.ref_path(other, kv))
    with pytest.raises(ts5hip.Ts5HipError, match="another model file"):
        ts5hip.ref_load(other, n, hp["n_vocab"], kv)
    ts5hip.ref_save(other, kv, got[:4])
    assert np.array_equal(ts5hip.ref_load(other, 4, hp["n_vocab"], kv), got[:4])
    with pytest.raises(ts5hip.Ts5HipError, match="fewer positions"):
        ts5hip.ref_load(other, 5, hp["n_vocab"], kv)
    with open(ts5hip.ref_path(other, kv), "wb") as f:
        f.write(b"NOTAREF!" + bytes(64))
    with pytest.raises(ts5hip.Ts5HipError, match="not a .ts5ref"):
        ts5hip.ref_load(other, 1, hp["n_vocab"], kv)
    assert not os.path.exists(ts5hip.ref_path(other, kv) + ".part")
