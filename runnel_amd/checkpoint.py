"""Real-tensor ingestion for the MoE block.

* ``SafeTensorStore``: every tensor of an MLX checkpoint directory (all
  ``*.safetensors`` shards), indexed from the shard headers and read by byte
  range, never a whole shard at once (bench/export_ornith_moe_layer.py:26-61;
  header checks of bench/runnel_bench/checkpoint.py:55-63).
* ``QuantSpec`` and ``load_moe_block``: one decoder layer's MoE block built
  from the checkpoint with its per-module quantization (config.json
  ``quantization``: defaults plus per-module overrides, resolved as
  bench/runnel_bench/checkpoint.py:104-121 does), ready for the packed
  gate/up transform.
* The reference's probe datasets: ``RNLMOE01`` (one layer's expert banks, 8
  selected experts, x and router weights; writer
  bench/export_ornith_moe_layer.py:18-19,118-168, reader
  native/src/fused_moe_probe.mm:44-54,539-591) and ``RNLQMV02`` (a QMV bank,
  x and the selected experts; native/src/quantized_qmv_probe.mm:39-49,
  312-352, reader bench/mlx_qmv_adapter.py:18-83): read, written, exported
  from a checkpoint and run through the HIP kernels.

Host code only: files are parsed here and the tensors handed to the GPU; the
arithmetic is librmoe.so's.
"""

from __future__ import annotations

import hashlib
import json
import math
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import NamedTuple

import numpy as np
import torch

from . import native

BF16 = torch.bfloat16

# --------------------------------------------------------------- safetensors

_DTYPES = {
    "U32": (np.dtype("<u4"), torch.int32),   # packed MLX-affine codes
    "I32": (np.dtype("<i4"), torch.int32),
    "BF16": (np.dtype("<u2"), BF16),
    "F16": (np.dtype("<f2"), torch.float16),
    "F32": (np.dtype("<f4"), torch.float32),
    "U8": (np.dtype("u1"), torch.uint8),
}
_MAX_HEADER = 100 * 1024 * 1024


class TensorInfo(NamedTuple):
    path: Path
    begin: int          # absolute byte offset in the file
    end: int
    shape: tuple
    dtype: str


def read_safetensors_header(path: Path) -> tuple[dict, int]:
    """(header dict, byte offset of the data section) of one shard."""
    with path.open("rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"invalid safetensors header in {path.name}")
        size = struct.unpack("<Q", raw)[0]
        if size <= 0 or size > _MAX_HEADER:
            raise ValueError(f"invalid safetensors header size in {path.name}")
        text = f.read(size)
        if len(text) != size:
            raise ValueError(f"truncated safetensors header in {path.name}")
    return json.loads(text), 8 + size


class SafeTensorStore:
    """The tensors of a checkpoint directory (or of one ``.safetensors``
    file), by name."""

    def __init__(self, root) -> None:
        root = Path(root)
        self.root = root if root.is_dir() else root.parent
        files = sorted(root.glob("*.safetensors")) if root.is_dir() else [root]
        if not files:
            raise FileNotFoundError(f"no *.safetensors files under {root}")
        self.entries: dict[str, TensorInfo] = {}
        for path in files:
            header, data = read_safetensors_header(path)
            size = path.stat().st_size
            for name, meta in header.items():
                if name == "__metadata__":
                    continue
                dtype = meta["dtype"]
                shape = tuple(int(d) for d in meta["shape"])
                b, e = (int(v) for v in meta["data_offsets"])
                # tensors of other dtypes are indexed too; reading them fails
                if dtype in _DTYPES:
                    nbytes = math.prod(shape) * _DTYPES[dtype][0].itemsize
                    if e - b != nbytes or b < 0 or data + e > size:
                        raise ValueError(f"tensor {name}: byte range [{b}, {e}) does not "
                                         f"match {dtype} {list(shape)} in {path.name}")
                if name in self.entries:
                    raise ValueError(f"tensor {name} appears in more than one shard")
                self.entries[name] = TensorInfo(path, data + b, data + e, shape, dtype)

    def __contains__(self, name: str) -> bool:
        return name in self.entries

    def names(self) -> list[str]:
        return sorted(self.entries)

    def info(self, name: str) -> TensorInfo:
        try:
            return self.entries[name]
        except KeyError:
            raise KeyError(f"tensor is missing: {name}") from None

    def _check_dtype(self, name: str, info: TensorInfo):
        if info.dtype not in _DTYPES:
            raise ValueError(f"unsupported tensor dtype {info.dtype} for {name}")
        return _DTYPES[info.dtype]

    def read(self, name: str) -> np.ndarray:
        """Host copy (numpy; BF16 as uint16 bit patterns)."""
        info = self.info(name)
        npt, _ = self._check_dtype(name, info)
        a = np.fromfile(info.path, dtype=npt, count=math.prod(info.shape), offset=info.begin)
        return a.reshape(info.shape)

    def tensor(self, name: str, device="cuda") -> torch.Tensor:
        """The tensor on `device` (U32 codes as int32, BF16 as bfloat16),
        read straight from its byte range into a pinned staging buffer."""
        info = self.info(name)
        _, tt = self._check_dtype(name, info)
        nbytes = info.end - info.begin
        pin = torch.device(device).type == "cuda" and torch.cuda.is_available()
        host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=pin)
        with info.path.open("rb") as f:
            f.seek(info.begin)
            got = f.readinto(memoryview(host.numpy()))
        if got != nbytes:
            raise ValueError(f"tensor {name} is truncated in {info.path.name}")
        t = host.view(tt).reshape(info.shape)
        return t if torch.device(device).type == "cpu" else t.to(device)

    def sha256(self, name: str) -> str:
        info = self.info(name)
        h = hashlib.sha256()
        with info.path.open("rb") as f:
            f.seek(info.begin)
            left = info.end - info.begin
            while left:
                chunk = f.read(min(left, 1 << 24))
                if not chunk:
                    raise ValueError(f"tensor {name} is truncated in {info.path.name}")
                h.update(chunk)
                left -= len(chunk)
        return h.hexdigest()


# --------------------------------------------------------------- quantization

class QuantSpec:
    """Per-module quantization of a checkpoint: config ``quantization`` (or
    ``quantization_config``) defaults, overridden by entries keyed by module
    name; a tensor name ending in ``.weight`` also finds its module's entry
    (bench/runnel_bench/checkpoint.py:113-121).  An entry of ``false`` marks
    a module kept in floating point."""

    def __init__(self, config: dict):
        q = config.get("quantization") or config.get("quantization_config") or {}
        self.bits = int(q.get("bits", 16))
        self.group_size = int(q.get("group_size", 64) or 64)
        self.mode = q.get("mode", "affine")
        self.overrides = {k: v for k, v in q.items() if isinstance(v, (dict, bool))}

    def of(self, name: str) -> tuple[int, int, str]:
        o = self.overrides.get(name)
        if o is None and name.endswith(".weight"):
            o = self.overrides.get(name[:-len(".weight")])
        if o is False:
            return 16, 0, "none"
        o = o if isinstance(o, dict) else {}
        return (int(o.get("bits", self.bits)), int(o.get("group_size", self.group_size) or 64),
                o.get("mode", self.mode))


def _load_config(store: SafeTensorStore, config) -> dict:
    if config is not None:
        return config
    path = store.root / "config.json"
    if not path.exists():
        raise FileNotFoundError(f"config.json not found under {store.root}")
    return json.loads(path.read_text(encoding="utf-8"))


def _layer_prefix(store: SafeTensorStore, layer: int) -> str:
    for p in (f"language_model.model.layers.{layer}.mlp", f"model.layers.{layer}.mlp"):
        if f"{p}.gate.weight" in store:
            return p
    raise KeyError(f"tensor is missing: language_model.model.layers.{layer}.mlp.gate.weight")


def _quantized(store, spec, module, out_dims, in_dims, device, experts=None):
    """(weight, scales, biases, bits, group_size) of an MLX-affine module,
    shapes checked against the config."""
    name = module + ".weight"
    bits, group, mode = spec.of(name)
    if mode != "affine":
        raise ValueError(f"{module}: quantization mode {mode!r} is not supported")
    if bits not in (4, 8):
        raise ValueError(f"{module}: expected 4- or 8-bit codes (config says {bits})")
    lead = () if experts is None else (experts,)
    want_w = (*lead, out_dims, in_dims * bits // 32)
    want_p = (*lead, out_dims, in_dims // group)
    for suffix, want, dt in ((".weight", want_w, ("U32", "I32")), (".scales", want_p, ("BF16",)),
                             (".biases", want_p, ("BF16",))):
        if module + suffix not in store:
            raise KeyError(f"tensor is missing: {module + suffix}")
        info = store.info(module + suffix)
        if info.shape != want or info.dtype not in dt:
            raise ValueError(f"{module + suffix}: expected {dt[0]} {list(want)} for {bits}-bit "
                             f"group-{group} codes, found {info.dtype} {list(info.shape)}")
    return (store.tensor(module + ".weight", device), store.tensor(module + ".scales", device),
            store.tensor(module + ".biases", device), bits, group)


def _gate(store, spec, module, out_dims, in_dims, device):
    """A router-style gate: quantized when the checkpoint has its scales,
    else a bf16 ``Linear``."""
    from .switch_layers import Linear, QuantizedLinear
    if module + ".scales" in store:
        w, s, b, bits, group = _quantized(store, spec, module, out_dims, in_dims, device)
        return QuantizedLinear(in_dims, out_dims, bits, group, weight=w, scales=s, biases=b)
    info = store.info(module + ".weight")
    if info.shape != (out_dims, in_dims) or info.dtype != "BF16":
        raise ValueError(f"{module}.weight: expected BF16 {[out_dims, in_dims]}, found "
                         f"{info.dtype} {list(info.shape)}")
    return Linear(in_dims, out_dims, weight=store.tensor(module + ".weight", device))


def load_moe_block(root_or_store, layer: int, device="cuda", config: dict | None = None,
                   fuse: bool = True):
    """The MoE block of decoder layer `layer` as a ``SparseMoeBlock`` on
    `device`: router ``gate`` (bf16 or quantized), ``switch_mlp`` (packed
    into ``FusedQuantizedSwitchGLU`` when `fuse`), ``shared_expert`` and
    ``shared_expert_gate``, sized from the config's ``text_config``."""
    from .moe import FusedQuantizedSwitchGLU, SparseMoeBlock
    from .switch_layers import MLP, QuantizedLinear, QuantizedSwitchLinear, SwitchGLU
    store = (root_or_store if isinstance(root_or_store, SafeTensorStore)
             else SafeTensorStore(root_or_store))
    cfg = _load_config(store, config)
    text = cfg.get("text_config", cfg)
    H = int(text["hidden_size"])
    E = int(text["num_experts"])
    K = int(text["num_experts_per_tok"])
    I = int(text["moe_intermediate_size"])
    Is = int(text.get("shared_expert_intermediate_size") or 0)
    norm = bool(text.get("norm_topk_prob", True))
    spec = QuantSpec(cfg)
    p = _layer_prefix(store, layer)

    sw = f"{p}.switch_mlp"
    projs = {}
    for proj, (o, i) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
        w, s, b, bits, group = _quantized(store, spec, f"{sw}.{proj}", o, i, device, experts=E)
        projs[proj] = QuantizedSwitchLinear(i, o, E, group_size=group, bits=bits, weight=w,
                                            scales=s, biases=b)
    bits = projs["gate_proj"].bits
    group = projs["gate_proj"].group_size
    shared = Is > 0 and f"{p}.shared_expert.gate_proj.weight" in store
    # modules are built on the meta device and their buffers replaced by
    # the checkpoint's tensors (no full-size zero banks on the GPU)
    blk = SparseMoeBlock(H, I, E, K, Is if shared else None, norm, bits, group, device="meta")
    blk.gate = _gate(store, spec, f"{p}.gate", E, H, device)
    sm = SwitchGLU(H, I, E, bits=bits, group_size=group, device="meta")
    sm.gate_proj, sm.up_proj, sm.down_proj = (projs["gate_proj"], projs["up_proj"],
                                              projs["down_proj"])
    blk.switch_mlp = sm
    if shared:
        mlp = MLP(H, Is, bits, group, device="meta")
        for proj, (o, i) in (("gate_proj", (Is, H)), ("up_proj", (Is, H)), ("down_proj", (H, Is))):
            w, s, b, pb, pg = _quantized(store, spec, f"{p}.shared_expert.{proj}", o, i, device)
            setattr(mlp, proj, QuantizedLinear(i, o, pb, pg, weight=w, scales=s, biases=b))
        blk.shared_expert = mlp
        blk.shared_expert_gate = _gate(store, spec, f"{p}.shared_expert_gate", 1, H, device)
    if fuse:
        blk.switch_mlp = FusedQuantizedSwitchGLU(blk.switch_mlp)
    return blk


def load_decoder_moe(root_or_store, layer: int, device="cuda", config: dict | None = None):
    """The MoE half of decoder layer `layer`: its ``post_attention_layernorm``
    (weight and the config's ``rms_norm_eps``) in front of the block, as a
    ``PostAttentionMoE`` computing ``h + mlp(norm(h))``."""
    from .moe import PostAttentionMoE
    from .switch_layers import RMSNorm
    store = (root_or_store if isinstance(root_or_store, SafeTensorStore)
             else SafeTensorStore(root_or_store))
    cfg = _load_config(store, config)
    text = cfg.get("text_config", cfg)
    H = int(text["hidden_size"])
    name = _layer_prefix(store, layer)[:-len(".mlp")] + ".post_attention_layernorm.weight"
    info = store.info(name)
    if info.shape != (H,) or info.dtype != "BF16":
        raise ValueError(f"{name}: expected BF16 [{H}], found {info.dtype} {list(info.shape)}")
    norm = RMSNorm(H, float(text.get("rms_norm_eps", 1e-6)), weight=store.tensor(name, device))
    return PostAttentionMoE(norm, load_moe_block(store, layer, device, cfg))


# ------------------------------------------------------------------ RNLMOE01

MOE_MAGIC = b"RNLMOE01"
MOE_HEADER = struct.Struct("<8s8I")
# x and router weights of an exported layer (export_ornith_moe_layer.py:134-140)
MOE_EXPORT_SEED = 0x4F524E495448
MOE_EXPORT_EXPERTS = (3, 17, 29, 42, 50, 61, 7, 55)


@dataclass
class MoeDataset:
    """One layer's routed expert banks with a fixed selection, input and
    router weights.  gate_up rows are [up; gate]."""
    bits: int
    selected: np.ndarray            # uint32 [k]
    gate_up: tuple                  # (u32 [E, 2I, H/vpw], u16 [E, 2I, H/64] x2)
    down: tuple                     # (u32 [E, H, I/vpw], u16 [E, H, I/64] x2)
    x: np.ndarray                   # bf16 bits [H]
    router: np.ndarray              # float32 [k]

    @property
    def total_experts(self) -> int:
        return self.gate_up[0].shape[0]

    @property
    def hidden(self) -> int:
        return self.down[0].shape[1]

    @property
    def inter(self) -> int:
        return self.gate_up[0].shape[1] // 2


def _bank_shapes(bits, E, rows, cols):
    vpw = 32 // bits
    return (E, rows, cols // vpw), (E, rows, cols // 64)


def read_rnlmoe01(path) -> MoeDataset:
    path = Path(path)
    raw = np.memmap(path, dtype=np.uint8, mode="r")
    if raw.size < MOE_HEADER.size:
        raise ValueError(f"fused MoE dataset is truncated: {path}")
    magic, version, bits, E, k, gu_rows, dn_rows, H, I = MOE_HEADER.unpack_from(raw[:MOE_HEADER.size].tobytes())
    if magic != MOE_MAGIC or version != 1:
        raise ValueError(f"not an RNLMOE01 version 1 dataset: {path}")
    if (bits not in (4, 8) or gu_rows != 2 * I or dn_rows != H or H % 64 or I % 64
            or H <= 0 or I <= 0 or E <= 0 or k <= 0):
        raise ValueError("fused MoE dataset header is inconsistent "
                         f"(bits {bits}, experts {E}, rows {gu_rows}/{dn_rows}, "
                         f"hidden {H}, inter {I})")
    off = MOE_HEADER.size

    def take(dtype, shape):
        nonlocal off
        n = math.prod(shape) * np.dtype(dtype).itemsize
        if off + n > raw.size:
            raise ValueError(f"fused MoE dataset is truncated: {path}")
        a = np.frombuffer(raw, dtype=dtype, count=math.prod(shape), offset=off).reshape(shape)
        off += n
        return a

    selected = take("<u4", (k,))
    gw, gp = _bank_shapes(bits, E, gu_rows, H)
    dw, dp = _bank_shapes(bits, E, dn_rows, I)
    gate_up = (take("<u4", gw), take("<u2", gp), take("<u2", gp))
    down = (take("<u4", dw), take("<u2", dp), take("<u2", dp))
    x = take("<u2", (H,))
    router = take("<f4", (k,))
    if off != raw.size:
        raise ValueError(f"fused MoE dataset has trailing bytes: {path}")
    if np.any(selected >= E):
        raise ValueError("selected expert is outside the dataset's bank")
    return MoeDataset(bits, selected, gate_up, down, x, router)


def write_rnlmoe01(path, ds: MoeDataset) -> None:
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("wb") as f:
        f.write(MOE_HEADER.pack(MOE_MAGIC, 1, ds.bits, ds.total_experts, len(ds.selected),
                                2 * ds.inter, ds.hidden, ds.hidden, ds.inter))
        for a, dt in ((ds.selected, "<u4"), (ds.gate_up[0], "<u4"), (ds.gate_up[1], "<u2"),
                      (ds.gate_up[2], "<u2"), (ds.down[0], "<u4"), (ds.down[1], "<u2"),
                      (ds.down[2], "<u2"), (ds.x, "<u2"), (ds.router, "<f4")):
            f.write(np.ascontiguousarray(a, dtype=dt).tobytes())


def _bf16_rne(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    special = ((u >> 23) & 0xFF) == 0xFF
    return np.where(special, u >> 16, (u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def export_inputs(hidden: int = 2048, k: int = 8):
    """The exporter's synthetic x (bf16 bits) and normalised router weights
    (export_ornith_moe_layer.py:134-140)."""
    rng = np.random.default_rng(MOE_EXPORT_SEED)
    x = rng.uniform(-1.0, 1.0, size=hidden).astype(np.float32)
    router = rng.uniform(0.5, 1.5, size=k).astype(np.float32)
    router /= np.sum(router, dtype=np.float32)
    return _bf16_rne(x), router


def export_rnlmoe01(root_or_store, layer: int, path, experts=MOE_EXPORT_EXPERTS,
                    manifest_path=None) -> dict:
    """Write layer `layer`'s routed banks as RNLMOE01 (the exporter of
    bench/export_ornith_moe_layer.py:80-168) and return its manifest."""
    store = (root_or_store if isinstance(root_or_store, SafeTensorStore)
             else SafeTensorStore(root_or_store))
    selected = [int(e) for e in experts]
    if len(selected) != 8 or len(set(selected)) != 8 or min(selected) < 0:
        raise ValueError("experts must contain eight unique non-negative indices")
    prefix = _layer_prefix(store, layer) + ".switch_mlp"
    t, hashes = {}, {}
    for proj in ("gate_proj", "up_proj", "down_proj"):
        for part in ("weight", "scales", "biases"):
            name = f"{prefix}.{proj}.{part}"
            t[(proj, part)] = store.read(name)
            hashes[name] = store.sha256(name)
    gw, uw, dw = t[("gate_proj", "weight")], t[("up_proj", "weight")], t[("down_proj", "weight")]
    if gw.ndim != 3 or uw.shape != gw.shape:
        raise ValueError("gate/up tensor shapes do not agree")
    if dw.ndim != 3:
        raise ValueError("down tensor is not an expert matrix")
    E, I, gpk = gw.shape
    H = dw.shape[1]
    if dw.shape[0] != E:
        raise ValueError("down tensor shape is inconsistent with gate/up rows")
    if max(selected) >= E:
        raise ValueError("selected expert is outside the checkpoint")
    bits = 32 * gpk // H
    if bits not in (4, 8) or gpk * (32 // bits) != H or dw.shape[2] != I * bits // 32:
        raise ValueError(f"cannot infer quantization bits from packed widths {gpk} / {dw.shape[2]}")
    x, router = export_inputs(H)
    ds = MoeDataset(
        bits, np.asarray(selected, np.uint32),
        tuple(np.concatenate((t[("up_proj", p)], t[("gate_proj", p)]), axis=1)
              for p in ("weight", "scales", "biases")),
        tuple(t[("down_proj", p)] for p in ("weight", "scales", "biases")), x, router)
    path = Path(path)
    write_rnlmoe01(path, ds)
    data = path.read_bytes()
    manifest = {
        "schema_version": 1, "model_name": store.root.name, "layer": layer, "bits": bits,
        "total_experts": E, "selected_experts": selected,
        "gate_up_shape": list(ds.gate_up[0].shape), "down_shape": list(dw.shape),
        "tensor_sha256": hashes, "output_sha256": hashlib.sha256(data).hexdigest(),
        "output_bytes": len(data),
        "note": "temporary derived artifact; model weights are not committed",
    }
    mpath = Path(manifest_path) if manifest_path else path.with_suffix(".manifest.json")
    mpath.write_text(json.dumps(manifest, indent=2, sort_keys=True) + "\n")
    return manifest


def _dev_u32(a, device):
    return torch.from_numpy(np.array(a, dtype=np.uint32).view(np.int32)).to(device)


def _dev_bf16(a, device):
    return torch.from_numpy(np.array(a, dtype=np.uint16).view(np.int16)).to(device).view(BF16)


def _dev_bank(bank, device):
    w, s, b = bank
    return _dev_u32(w, device), _dev_bf16(s, device), _dev_bf16(b, device)


def run_rnlmoe01(ds: MoeDataset, device="cuda") -> torch.Tensor:
    """The probe's two-stage MoE on the dataset: the selected experts on x,
    combined with the router weights -> bf16 [hidden] (rmoe_switch_combine)."""
    gu = _dev_bank(ds.gate_up, device)
    dn = _dev_bank(ds.down, device)
    gq = native.qweight_struct(*gu, ds.bits)
    dq = native.qweight_struct(*dn, ds.bits)
    x = _dev_bf16(ds.x[None, :], device)
    idx = torch.from_numpy(np.array(ds.selected, np.int64).astype(np.int32)[None, :]).to(device)
    w = torch.from_numpy(np.array(ds.router, np.float32)[None, :]).to(device)
    out = native.switch_combine(x, idx, w, gq, dq)
    return out[0]


# ------------------------------------------------------------------ RNLQMV02

QMV_MAGIC = b"RNLQMV02"
QMV_HEADER = struct.Struct("<8sIIIIIIII")


@dataclass
class QmvDataset:
    """A quantized bank of rows_per_expert-row experts, x, and the selected
    experts whose rows form the output (in selection order)."""
    bits: int
    output_size: int
    rows_per_expert: int
    group_size: int
    weights: np.ndarray             # uint32 [bank_rows, K/vpw]
    scales: np.ndarray              # bf16 bits [bank_rows, K/group]
    biases: np.ndarray
    x: np.ndarray                   # bf16 bits [K]
    selected: np.ndarray            # uint32 [n]

    @property
    def bank_rows(self) -> int:
        return self.weights.shape[0]

    @property
    def reduction_size(self) -> int:
        return self.x.shape[0]


def read_rnlqmv02(path) -> QmvDataset:
    path = Path(path)
    raw = path.read_bytes()
    if len(raw) < QMV_HEADER.size:
        raise ValueError("QMV dataset is truncated")
    magic, version, bits, out, bank, rpe, K, group, n_sel = QMV_HEADER.unpack_from(raw)
    if magic != QMV_MAGIC or version != 2:
        raise ValueError("unsupported QMV dataset header")
    if bits not in (4, 8) or group <= 0 or K % (32 // bits) or K % group:
        raise ValueError("QMV dataset shape is incompatible with packing")
    if rpe == 0 or bank % rpe or out != n_sel * rpe:
        raise ValueError("QMV dataset expert layout is inconsistent")
    off = QMV_HEADER.size

    def take(dtype, count):
        nonlocal off
        n = count * np.dtype(dtype).itemsize
        if off + n > len(raw):
            raise ValueError("QMV dataset is truncated")
        a = np.frombuffer(raw, dtype=dtype, count=count, offset=off)
        off += n
        return a

    w = take("<u4", bank * K // (32 // bits)).reshape(bank, -1)
    s = take("<u2", bank * K // group).reshape(bank, -1)
    b = take("<u2", bank * K // group).reshape(bank, -1)
    x = take("<u2", K)
    sel = take("<u4", n_sel)
    if off != len(raw):
        raise ValueError("QMV dataset contains trailing bytes")
    if np.any(sel >= bank // rpe):
        raise ValueError("selected expert is outside the QMV bank")
    return QmvDataset(bits, out, rpe, group, w, s, b, x, sel)


def write_rnlqmv02(path, ds: QmvDataset) -> None:
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("wb") as f:
        f.write(QMV_HEADER.pack(QMV_MAGIC, 2, ds.bits, ds.output_size, ds.bank_rows,
                                ds.rows_per_expert, ds.reduction_size, ds.group_size,
                                len(ds.selected)))
        for a, dt in ((ds.weights, "<u4"), (ds.scales, "<u2"), (ds.biases, "<u2"),
                      (ds.x, "<u2"), (ds.selected, "<u4")):
            f.write(np.ascontiguousarray(a, dtype=dt).tobytes())


def run_rnlqmv02(ds: QmvDataset, device="cuda") -> torch.Tensor:
    """The QMV of the dataset: output row r is bank row
    selected[r // rpe] * rpe + r % rpe (quantized_qmv_probe.mm:355-363),
    as float32 [output_size] (rmoe_gather_qmm with fp32 output)."""
    if ds.group_size != 64:
        raise ValueError(f"group size {ds.group_size} is not supported (64 only)")
    E = ds.bank_rows // ds.rows_per_expert
    w = _dev_u32(ds.weights, device).reshape(E, ds.rows_per_expert, -1)
    s = _dev_bf16(ds.scales, device).reshape(E, ds.rows_per_expert, -1)
    b = _dev_bf16(ds.biases, device).reshape(E, ds.rows_per_expert, -1)
    x = _dev_bf16(ds.x[None, :], device)
    rhs = torch.from_numpy(np.asarray(ds.selected, np.int64).astype(np.int32)).to(device)
    lhs = torch.zeros_like(rhs)
    y = native.gather_qmm(x, w, s, b, ds.bits, 64, rhs_indices=rhs, lhs_indices=lhs,
                          out_dtype=torch.float32)
    return y.reshape(-1)
