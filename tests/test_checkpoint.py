"""Real-tensor ingestion without a GPU: the safetensors reader against the
`safetensors` package (an independent implementation) and against hand-built
files with the reference test's checkpoint layout; the per-module
quantization rule; the RNLQMV02 writer against the SHA-256 the reference
recorded for its own dataset files; RNLMOE01 round trips and the exporter;
a checkpoint layer loaded into the block modules and validated by the C ABI
(host-only)."""

import hashlib
import json
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import moe_ref as M
from runnel_amd import checkpoint as C

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
DT = {"U32": "<u4", "I32": "<i4", "BF16": "<u2", "F32": "<f4", "F64": "<f8"}


def write_safetensors(path: Path, tensors: dict, metadata=None, pad_to=8):
    """A safetensors file from {name: (dtype, numpy array)} (header JSON,
    8-byte little-endian length, data in header order)."""
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, (dtype, arr) in tensors.items():
        raw = np.ascontiguousarray(arr, dtype=DT[dtype]).tobytes()
        header[name] = {"dtype": dtype, "shape": list(np.shape(arr)),
                        "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % pad_to)
    path.write_bytes(struct.pack("<Q", len(text)) + text + b"".join(blobs))


def test_store_matches_the_safetensors_package(tmp_path):
    st = pytest.importorskip("safetensors.torch")
    g = torch.Generator().manual_seed(0)
    ts = {"a.weight": torch.randint(-2**31, 2**31 - 1, (4, 6), generator=g, dtype=torch.int32),
          "a.scales": torch.randn(4, 2, generator=g).to(torch.bfloat16),
          "b": torch.randn(3, generator=g)}
    st.save_file(ts, str(tmp_path / "m-00001-of-00002.safetensors"), metadata={"format": "mlx"})
    st.save_file({"c": torch.randn(2, 2, generator=g).to(torch.bfloat16)},
                 str(tmp_path / "m-00002-of-00002.safetensors"))
    store = C.SafeTensorStore(tmp_path)
    assert store.names() == ["a.scales", "a.weight", "b", "c"]
    from safetensors import safe_open
    for f in sorted(tmp_path.glob("*.safetensors")):
        with safe_open(str(f), framework="pt") as h:
            for name in h.keys():
                want = h.get_tensor(name)
                got = store.tensor(name, device="cpu")
                assert got.dtype == want.dtype and torch.equal(got, want)
                raw = store.read(name)
                assert raw.tobytes() == want.contiguous().view(torch.uint8).numpy().tobytes()
                assert store.sha256(name) == hashlib.sha256(raw.tobytes()).hexdigest()


def test_store_reads_u32_codes_and_rejects_bad_files(tmp_path):
    codes = np.arange(12, dtype=np.uint32).reshape(3, 4) * 0x01010101
    write_safetensors(tmp_path / "x.safetensors",
                      {"w": ("U32", codes), "d": ("F64", np.zeros(2))})
    store = C.SafeTensorStore(tmp_path / "x.safetensors")
    assert np.array_equal(store.read("w"), codes)
    assert torch.equal(store.tensor("w", "cpu"), torch.from_numpy(codes.view(np.int32)))
    with pytest.raises(ValueError, match="unsupported tensor dtype F64 for d"):
        store.read("d")
    with pytest.raises(KeyError, match="tensor is missing: nope"):
        store.read("nope")
    bad = tmp_path / "bad"
    bad.mkdir()
    (bad / "t.safetensors").write_bytes(b"\x01\x02")
    with pytest.raises(ValueError, match="invalid safetensors header"):
        C.SafeTensorStore(bad)
    (bad / "t.safetensors").write_bytes(struct.pack("<Q", 1 << 40))
    with pytest.raises(ValueError, match="header size"):
        C.SafeTensorStore(bad)
    # a byte range that does not match the declared shape
    hdr = json.dumps({"w": {"dtype": "U32", "shape": [2, 2], "data_offsets": [0, 12]}}).encode()
    (bad / "t.safetensors").write_bytes(struct.pack("<Q", len(hdr)) + hdr + bytes(12))
    with pytest.raises(ValueError, match="does not match"):
        C.SafeTensorStore(bad)
    with pytest.raises(FileNotFoundError):
        C.SafeTensorStore(tmp_path / "empty_dir_missing")


def test_quant_spec_resolution():
    """Defaults, a module override found by module or tensor name (the rule
    of bench/runnel_bench/checkpoint.py:113-121), and an unquantized module."""
    cfg = {"quantization": {"bits": 4, "group_size": 64, "mode": "affine",
                            "model.layers.0.mlp.gate": {"bits": 8, "group_size": 64},
                            "model.layers.0.mlp.shared_expert_gate": False}}
    q = C.QuantSpec(cfg)
    assert q.of("model.layers.0.mlp.switch_mlp.up_proj.weight") == (4, 64, "affine")
    assert q.of("model.layers.0.mlp.gate") == (8, 64, "affine")
    assert q.of("model.layers.0.mlp.gate.weight") == (8, 64, "affine")
    assert q.of("model.layers.0.mlp.shared_expert_gate.weight")[0] == 16
    assert C.QuantSpec({"quantization_config": {"bits": 8}}).of("x.weight") == (8, 64, "affine")


def write_checkpoint(root: Path, L: M.Layer, layer: int = 0, bits: int = 8, extra=None):
    """An MLX-style checkpoint directory holding one MoE layer of the
    oracle layer `L` (the config and tensor names of the reference test's
    fixture, tests/test_checkpoint.py there): unpacked [up; gate] banks,
    quantized or bf16 gates, a per-module 8-bit override for quantized
    gates on a 4-bit model."""
    root.mkdir(parents=True, exist_ok=True)
    I, H, E = L.inter, L.hidden, L.experts
    q = {"bits": bits, "group_size": 64, "mode": "affine"}
    p = f"language_model.model.layers.{layer}.mlp"
    t = {}

    def bank(name, qw, rows=None, expert_axis=True):
        w, s, b = qw.w, qw.scales, qw.biases
        if rows is not None:
            w, s, b = w[:, rows], s[:, rows], b[:, rows]
        if not expert_axis:
            w, s, b = w[0], s[0], b[0]
        t[name + ".weight"] = ("U32", w)
        t[name + ".scales"] = ("BF16", s)
        t[name + ".biases"] = ("BF16", b)

    def gate(name, g):
        if isinstance(g, M.QWeight):
            bank(name, g, expert_axis=False)
            q[name] = {"bits": g.bits, "group_size": 64}
        else:
            t[name + ".weight"] = ("BF16", g.reshape(-1, H))

    gate(f"{p}.gate", L.router_w)
    bank(f"{p}.switch_mlp.up_proj", L.gate_up, slice(0, I))
    bank(f"{p}.switch_mlp.gate_proj", L.gate_up, slice(I, 2 * I))
    bank(f"{p}.switch_mlp.down_proj", L.down)
    Is = 0
    if L.shared_gate_up is not None:
        Is = L.shared_inter
        bank(f"{p}.shared_expert.up_proj", L.shared_gate_up, slice(0, Is), expert_axis=False)
        bank(f"{p}.shared_expert.gate_proj", L.shared_gate_up, slice(Is, 2 * Is),
             expert_axis=False)
        bank(f"{p}.shared_expert.down_proj", L.shared_down, expert_axis=False)
        gate(f"{p}.shared_expert_gate", L.shared_gate_w)
    t.update(extra or {})
    names = sorted(t)
    half = len(names) // 2
    write_safetensors(root / "model-00001-of-00002.safetensors", {n: t[n] for n in names[:half]},
                      metadata={"format": "mlx"})
    write_safetensors(root / "model-00002-of-00002.safetensors", {n: t[n] for n in names[half:]})
    cfg = {"model_type": "qwen3_5_moe", "quantization": q,
           "text_config": {"hidden_size": H, "num_experts": E, "num_experts_per_tok": L.top_k,
                           "moe_intermediate_size": I, "shared_expert_intermediate_size": Is,
                           "norm_topk_prob": L.norm_topk_prob, "num_hidden_layers": layer + 1}}
    (root / "config.json").write_text(json.dumps(cfg))


@pytest.mark.parametrize("router_bits", [None, 8])
@pytest.mark.parametrize("bits", [8, 4])
def test_load_moe_block_from_checkpoint(tmp_path, monkeypatch, bits, router_bits):
    """Every buffer equals the checkpoint's bytes, gate/up are packed
    [up; gate], the gates take the format the checkpoint has, and the C ABI
    accepts the layer it describes (host tensors are refused for the kernels;
    the device check is lifted to describe them here)."""
    from runnel_amd import FusedQuantizedSwitchGLU, Linear, QuantizedLinear
    L = M.make_layer(3, hidden=256, inter=128, experts=8, top_k=2, bits=bits,
                     router_bits=router_bits)
    write_checkpoint(tmp_path, L, layer=2, bits=bits)
    blk = C.load_moe_block(tmp_path, 2, device="cpu")
    assert blk.top_k == 2 and blk.num_experts == 8
    sm = blk.switch_mlp
    assert isinstance(sm, FusedQuantizedSwitchGLU) and sm.bits == bits
    assert np.array_equal(sm.weight.numpy().view(np.uint32), L.gate_up.w)
    assert np.array_equal(sm.scales.view(torch.int16).numpy().view(np.uint16), L.gate_up.scales)
    assert np.array_equal(sm.down_proj.weight.numpy().view(np.uint32), L.down.w)
    gate_type = Linear if router_bits is None else QuantizedLinear
    assert type(blk.gate) is gate_type and type(blk.shared_expert_gate) is gate_type
    if router_bits:
        assert blk.gate.bits == 8
        assert np.array_equal(blk.gate.weight.numpy().view(np.uint32), L.router_w.w[0])
    se = blk.shared_expert
    assert np.array_equal(se.down_proj.weight.numpy().view(np.uint32), L.shared_down.w[0])
    with pytest.raises(ValueError, match="GPU tensors"):
        blk.layer_handle()
    from runnel_amd import native
    monkeypatch.setattr(native, "_require_cuda", lambda *t: None)
    h = blk.layer_handle()
    assert h is not None and h.struct.experts == 8 and h.struct.hidden == 256
    assert (h.struct.router_q.w is not None) == (router_bits is not None)


def test_load_decoder_moe_reads_the_post_attention_norm(tmp_path, monkeypatch):
    from runnel_amd import PostAttentionMoE, native
    monkeypatch.setattr(native, "_require_cuda", lambda *t: None)  # describe host tensors
    L = M.make_layer(5, hidden=256, inter=128, experts=8, top_k=2, bits=8)
    nw = M.f32_to_bf16(np.linspace(0.5, 1.5, 256).astype(np.float32))
    write_checkpoint(tmp_path, L, layer=1,
                     extra={"language_model.model.layers.1.post_attention_layernorm.weight":
                            ("BF16", nw)})
    cfg = json.loads((tmp_path / "config.json").read_text())
    cfg["text_config"]["rms_norm_eps"] = 1e-5
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    step = C.load_decoder_moe(tmp_path, 1, device="cpu")
    assert isinstance(step, PostAttentionMoE)
    norm = step.post_attention_layernorm
    assert norm.eps == pytest.approx(1e-5)
    assert np.array_equal(norm.weight.view(torch.int16).numpy().view(np.uint16), nw)
    h = step.layer_handle()
    assert h.struct.post_norm_w == norm.weight.data_ptr()
    assert h.struct.norm_eps == pytest.approx(1e-5)
    assert step.mlp.layer_handle().struct.post_norm_w is None   # the plain block's handle


def test_load_moe_block_reports_missing_and_misshaped_tensors(tmp_path):
    L = M.make_layer(4, hidden=256, inter=128, experts=8, top_k=2, bits=8)
    write_checkpoint(tmp_path / "a", L)
    cfg = json.loads((tmp_path / "a" / "config.json").read_text())
    cfg["text_config"]["moe_intermediate_size"] = 64
    with pytest.raises(ValueError, match="expected U32"):
        C.load_moe_block(tmp_path / "a", 0, device="cpu", config=cfg)
    with pytest.raises(KeyError, match="tensor is missing"):
        C.load_moe_block(tmp_path / "a", 5, device="cpu")
    cfg = json.loads((tmp_path / "a" / "config.json").read_text())
    cfg["quantization"]["bits"] = 4
    with pytest.raises(ValueError, match="4-bit group-64"):
        C.load_moe_block(tmp_path / "a", 0, device="cpu", config=cfg)


@pytest.mark.parametrize("case", GOLDEN["mlx_qmv"], ids=lambda c: Path(c["source"]).stem)
def test_rnlqmv02_writer_reproduces_recorded_dataset(case, tmp_path):
    """The package's writer, fed the reference probe's dataset, produces the
    file whose SHA-256 the reference recorded; its reader returns every
    array unchanged."""
    bits = case["bits"]
    o = M.qmv_dataset(bits, case["output_size"], case["reduction_size"], case["group"])
    ds = C.QmvDataset(bits, case["output_size"], case["output_size"], case["group"], o["w"],
                      o["scales"], o["biases"], o["x"], o["selected"])
    path = tmp_path / "ds.bin"
    C.write_rnlqmv02(path, ds)
    assert hashlib.sha256(path.read_bytes()).hexdigest() == case["dataset_sha256"]
    back = C.read_rnlqmv02(path)
    for f in ("weights", "scales", "biases", "x", "selected"):
        assert np.array_equal(getattr(back, f), getattr(ds, f))
    assert (back.bits, back.output_size, back.rows_per_expert, back.group_size) == \
        (bits, case["output_size"], case["output_size"], case["group"])


def test_rnlqmv02_reader_rejects_bad_files(tmp_path):
    o = M.qmv_dataset(8, 128, 256, 64, bank_rows=512, rows_per_expert=64, selected=(1, 6))
    ds = C.QmvDataset(8, 128, 64, 64, o["w"], o["scales"], o["biases"], o["x"], o["selected"])
    p = tmp_path / "q.bin"
    C.write_rnlqmv02(p, ds)
    good = p.read_bytes()
    back = C.read_rnlqmv02(p)
    assert back.bank_rows == 512 and list(back.selected) == [1, 6]
    p.write_bytes(good[:-1])
    with pytest.raises(ValueError, match="truncated"):
        C.read_rnlqmv02(p)
    p.write_bytes(good + b"\0")
    with pytest.raises(ValueError, match="trailing"):
        C.read_rnlqmv02(p)
    p.write_bytes(b"RNLQMV01" + good[8:])
    with pytest.raises(ValueError, match="unsupported QMV dataset header"):
        C.read_rnlqmv02(p)
    bad = bytearray(good)
    bad[-4:] = struct.pack("<I", 8)                 # expert 8 of an 8-expert bank
    p.write_bytes(bytes(bad))
    with pytest.raises(ValueError, match="outside"):
        C.read_rnlqmv02(p)


def _moe_dataset(bits, E=6, H=256, I=128, seed=0):
    L = M.make_layer(seed, hidden=H, inter=I, experts=E, top_k=2, bits=bits, shared=False)
    x, router = C.export_inputs(H)
    return C.MoeDataset(bits, np.array([4, 1, 0, 5, 2, 3, 1, 0], np.uint32)[:8] % E,
                        (L.gate_up.w, L.gate_up.scales, L.gate_up.biases),
                        (L.down.w, L.down.scales, L.down.biases), x, router)


@pytest.mark.parametrize("bits", [8, 4])
def test_rnlmoe01_round_trip_and_layout(tmp_path, bits):
    """Header fields and section order of export_ornith_moe_layer.py:142-168:
    magic, version 1, bits, experts, 8 selected, 2I and H rows per expert,
    hidden, intermediate; then selected, gate/up words, scales, biases, down
    words, scales, biases, x, router."""
    ds = _moe_dataset(bits)
    p = tmp_path / "l.bin"
    C.write_rnlmoe01(p, ds)
    raw = p.read_bytes()
    assert struct.unpack_from("<8s8I", raw) == (b"RNLMOE01", 1, bits, 6, 8, 256, 256, 256, 128)
    vpw = 32 // bits
    n_gu = 6 * 256 * (256 // vpw) * 4 + 2 * 6 * 256 * 4 * 2
    n_dn = 6 * 256 * (128 // vpw) * 4 + 2 * 6 * 256 * 2 * 2
    assert len(raw) == 40 + 8 * 4 + n_gu + n_dn + 256 * 2 + 8 * 4
    assert raw[-32:] == ds.router.astype("<f4").tobytes()
    back = C.read_rnlmoe01(p)
    assert back.bits == bits and back.total_experts == 6 and back.hidden == 256
    for a, b in zip((*back.gate_up, *back.down, back.x, back.router, back.selected),
                    (*ds.gate_up, *ds.down, ds.x, ds.router, ds.selected)):
        assert np.array_equal(a, b)
    p.write_bytes(raw[:-4])
    with pytest.raises(ValueError, match="truncated"):
        C.read_rnlmoe01(p)
    p.write_bytes(raw + b"\0\0")
    with pytest.raises(ValueError, match="trailing"):
        C.read_rnlmoe01(p)
    bad = bytearray(raw)
    bad[24:28] = struct.pack("<I", 200)          # gate/up rows != 2 * inter
    p.write_bytes(bytes(bad))
    with pytest.raises(ValueError, match="inconsistent"):
        C.read_rnlmoe01(p)


def test_export_inputs_are_the_exporters():
    """x is uniform(-1, 1) rounded to bf16 and the router weights are
    uniform(0.5, 1.5) normalised in float32, both from PCG64 seeded
    0x4F524E495448: bf16 values, in range, router sums to one."""
    x, r = C.export_inputs(2048)
    xf = M.bf16_to_f32(x)
    assert x.dtype == np.uint16 and x.shape == (2048,)
    assert np.all(np.abs(xf) <= 1.0) and np.abs(xf).max() > 0.99
    rng = np.random.default_rng(0x4F524E495448)
    want = rng.uniform(-1.0, 1.0, size=2048).astype(np.float32)
    assert np.array_equal(x, M.f32_to_bf16(want))
    assert r.dtype == np.float32 and abs(float(r.sum(dtype=np.float64)) - 1.0) < 1e-6
    assert np.all((r > 0.5 / 8 / 1.5) & (r < 1.5 / 8 / 0.5))


@pytest.mark.parametrize("bits", [8, 4])
def test_export_rnlmoe01_from_checkpoint(tmp_path, bits):
    """The exporter reads the switch_mlp tensors, packs [up; gate], writes
    the dataset and a manifest whose hashes are those of the tensors' bytes
    and of the file."""
    L = M.make_layer(9, hidden=256, inter=128, experts=64, top_k=2, bits=bits, shared=False)
    write_checkpoint(tmp_path / "ckpt", L, layer=1, bits=bits)
    out = tmp_path / "cache" / "layer-1.bin"
    man = C.export_rnlmoe01(tmp_path / "ckpt", 1, out)
    ds = C.read_rnlmoe01(out)
    assert ds.bits == bits and list(ds.selected) == list(C.MOE_EXPORT_EXPERTS)
    assert np.array_equal(ds.gate_up[0], L.gate_up.w) and np.array_equal(ds.down[2], L.down.biases)
    assert man["output_sha256"] == hashlib.sha256(out.read_bytes()).hexdigest()
    store = C.SafeTensorStore(tmp_path / "ckpt")
    name = "language_model.model.layers.1.mlp.switch_mlp.up_proj.weight"
    assert man["tensor_sha256"][name] == hashlib.sha256(store.read(name).tobytes()).hexdigest()
    assert json.loads(out.with_suffix(".manifest.json").read_text()) == man
    with pytest.raises(ValueError, match="eight unique"):
        C.export_rnlmoe01(tmp_path / "ckpt", 1, out, experts=(1, 2, 3))
    with pytest.raises(ValueError, match="outside the checkpoint"):
        C.export_rnlmoe01(tmp_path / "ckpt", 1, out, experts=(1, 2, 3, 4, 5, 6, 7, 64))
