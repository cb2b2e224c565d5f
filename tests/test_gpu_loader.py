"""ut_model_load_dir: converted safetensors checkpoints streamed from disk
into HBM (read_qtensor, ShardedModelReader; undertow-io/src/reader.rs),
against the same tensors handed over by ut_model_set_tensor and against the
reference's transformers golden."""
import json
import struct

import numpy as np
import pytest

from models import C1, checkpoint, gpu_model, prompt_ids, write_converted
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def fresh_model(ctx, ck):
    import undertow_amd as U
    from models import CFG_KEYS
    return U.Model(ctx, {k: getattr(ck.spec, k) for k in CFG_KEYS})


def write_safetensors(path, entries):
    """A minimal safetensors writer for test fixtures: entries of
    (name, dtype string, shape, raw bytes)."""
    hdr, off, blobs = {}, 0, []
    for name, dt, shape, raw in entries:
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
        blobs.append(raw)
    h = json.dumps(hdr, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    path.write_bytes(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def test_sharded_int4_checkpoint_loads_bit_identical(ctx, tmp_path):
    ck = checkpoint(C1, fmt="int4")
    write_converted(ck, tmp_path, expert_layers=[1, 2])
    m = fresh_model(ctx, ck)
    nbytes = m.load_dir(tmp_path)
    total = sum(p.nbytes + (0 if s is None else s.nbytes) for _, _, _, p, s in ck.tensors())
    assert nbytes == total
    ref = gpu_model(ctx, ck)
    prompt = prompt_ids(16, C1["vocab_size"])
    assert np.array_equal(m.forward(prompt), ref.forward(prompt))
    assert m.generate_mtp(prompt, 16, depth=1) == ref.generate_mtp(prompt, 16, depth=1)


def test_single_file_f32_matches_transformers_golden(ctx, tmp_path, golden_dir):
    ck = checkpoint()
    (tmp_path / "model.safetensors").write_bytes(ck.safetensors_bytes())
    m = fresh_model(ctx, ck)
    m.load_dir(tmp_path)
    ref = json.loads((golden_dir / "oracle-tiny" / "reference.json").read_text())
    logits = m.forward(ref["full_ids"])
    assert np.abs(logits - np.asarray(ref["tf_logits"], np.float32)).max() < 1e-3
    assert logits.argmax(1).tolist() == ref["tf_pred"]


def test_bf16_and_f16_tensors_widen_exactly(ctx, tmp_path):
    """Plain BF16 / F16 tensors load as their exact f32 values."""
    import torch
    ck = checkpoint()
    entries, expect = [], {}
    for i, (name, fmt, shape, payload, scales) in enumerate(ck.tensors()):
        a = np.frombuffer(payload.tobytes(), np.float32).reshape(shape)
        if i % 3 == 1:
            t = torch.from_numpy(a.copy()).to(torch.bfloat16)
            entries.append((name, "BF16", shape, t.view(torch.int16).numpy().tobytes()))
            expect[name] = t.float().numpy()
        elif i % 3 == 2:
            h = a.astype(np.float16)
            entries.append((name, "F16", shape, h.tobytes()))
            expect[name] = h.astype(np.float32)
        else:
            entries.append((name, "F32", shape, a.tobytes()))
            expect[name] = a
    write_safetensors(tmp_path / "model.safetensors", entries)
    m = fresh_model(ctx, ck)
    m.load_dir(tmp_path)
    ref = fresh_model(ctx, ck)
    for name, fmt, shape, payload, scales in ck.tensors():
        ref.set_tensor(name, O.F32, expect[name], None, shape)
    ref.finalize()
    ids = prompt_ids(12, ck.spec.vocab_size)
    assert np.array_equal(m.forward(ids), ref.forward(ids))


def test_bad_checkpoints_are_rejected(ctx, tmp_path):
    import undertow_amd as U
    ck = checkpoint(C1, fmt="int4")
    m = fresh_model(ctx, ck)
    with pytest.raises(U.UtError) as ei:
        m.load_dir(tmp_path / "nowhere")
    assert ei.value.code == U.runtime.UT_ERR_IO
    # a tensor the config needs is missing
    ts = [t for t in ck.tensors() if t[0] != "model.norm.weight"]
    (tmp_path / "model.safetensors").write_bytes(O.Checkpoint.from_tensors(ck.spec, ts).safetensors_bytes())
    with pytest.raises(U.UtError) as ei:
        fresh_model(ctx, ck).load_dir(tmp_path)
    assert ei.value.code == U.runtime.UT_ERR_NOT_FOUND and "model.norm.weight" in str(ei.value)
    # data_offsets past the end of the file
    blob = ck.safetensors_bytes()
    (tmp_path / "model.safetensors").write_bytes(blob[:-100])
    with pytest.raises(U.UtError) as ei:
        fresh_model(ctx, ck).load_dir(tmp_path)
    assert ei.value.code == U.runtime.UT_ERR_FORMAT and "inconsistent" in str(ei.value)
    # a payload whose size is neither int8 nor int4 for the shape
    bad = []
    for name, fmt, shape, payload, scales in ck.tensors():
        if name == "lm_head.weight":
            payload = payload.reshape(-1)[:-1]
            bad.append((name, "U8", (payload.size,), payload.tobytes()))
            bad.append((name + ".scales", "F32", scales.shape, scales.tobytes()))
        elif fmt == O.F32:
            bad.append((name, "F32", shape, payload.tobytes()))
        else:
            bad.append((name, "U8", (payload.size,), payload.tobytes()))
            bad.append((name + ".scales", "F32", scales.shape, scales.tobytes()))
    write_safetensors(tmp_path / "model.safetensors", bad)
    with pytest.raises(U.UtError) as ei:
        fresh_model(ctx, ck).load_dir(tmp_path)
    assert ei.value.code == U.runtime.UT_ERR_FORMAT and "lm_head.weight" in str(ei.value)
    # a header that is not JSON
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", 8) + b"{nojson ")
    with pytest.raises(U.UtError) as ei:
        fresh_model(ctx, ck).load_dir(tmp_path)
    assert ei.value.code == U.runtime.UT_ERR_FORMAT


def test_bf16_scales_and_any_payload_dtype(ctx, tmp_path):
    """read_qtensor (reader.rs:403-444) takes the payload raw whatever its
    dtype and reads `.scales` through read_f32, which widens BF16 / F16: a
    converted checkpoint with 16-bit scales and I8 payloads loads, resident
    and behind the HBM tier, as the same model with the widened scales."""
    import torch
    ck = checkpoint(C1, fmt="int4")
    entries, ref = [], fresh_model(ctx, ck)
    for i, (name, fmt, shape, payload, scales) in enumerate(ck.tensors()):
        if fmt == O.F32:
            entries.append((name, "F32", shape, payload.tobytes()))
            ref.set_tensor(name, fmt, payload, None, shape)
            continue
        if i % 2:
            t = torch.from_numpy(np.ascontiguousarray(scales, np.float32)).to(torch.bfloat16)
            raw, wide, dt = t.view(torch.int16).numpy().tobytes(), t.float().numpy(), "BF16"
        else:
            h = np.asarray(scales, np.float32).astype(np.float16)
            raw, wide, dt = h.tobytes(), h.astype(np.float32), "F16"
        entries.append((name, "I8" if i % 3 == 0 else "U8", (payload.size,), payload.tobytes()))
        entries.append((name + ".scales", dt, (shape[0],), raw))
        ref.set_tensor(name, fmt, payload, wide, shape)
    ref.finalize()
    write_safetensors(tmp_path / "model.safetensors", entries)
    ids = prompt_ids(12, ck.spec.vocab_size)
    want = ref.forward(ids)
    m = fresh_model(ctx, ck)
    m.load_dir(tmp_path)
    assert np.array_equal(m.forward(ids), want)
    H, I = ck.spec.hidden_size, ck.spec.moe_intermediate_size
    tiered = fresh_model(ctx, ck)
    tiered.load_dir_tiered(tmp_path, hbm_budget_bytes=2 * (2 * I * (H // 2) + H * (I // 2) + (2 * I + H) * 4))
    assert np.array_equal(tiered.forward(ids), want)
    assert tiered.store_stats()["misses"] > 0
