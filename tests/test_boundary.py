"""The drop-in boundary without a GPU: the C ABI loads and exports what
include/rmoe.h declares, rejects bad arguments on the host before anything
is launched, and the torch-side modules keep the surface, validation and
error messages of src/runnel/mlx.py.  No test here launches a kernel."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from runnel_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
FAKE = 0x100000  # an aligned, never-dereferenced address


def declared_functions():
    text = (ROOT / "include" / "rmoe.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(rmoe_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.EXPORTED)
    assert lib.rmoe_abi_version() == _lib.ABI_VERSION


def _qw(bits=8, experts=4, rows=128, cols=256, ptr=FAKE):
    return _lib.QWeight(ptr, ptr, ptr, experts, rows, cols, bits, 64)


def _layer(bits=8, E=4, H=256, I=64, K=2, shared=True):
    return _lib.Layer(H, I, I if shared else 0, E, K, 1, FAKE, FAKE if shared else None,
                      _qw(bits, E, 2 * I, H), _qw(bits, E, H, I),
                      _qw(bits, 1, 2 * I, H) if shared else _lib.QWeight(),
                      _qw(bits, 1, H, I) if shared else _lib.QWeight())


def test_validate_layer_accepts_and_rejects():
    lib = _lib.load()
    assert lib.rmoe_validate_layer(ctypes.byref(_layer())) == _lib.RMOE_OK
    assert lib.rmoe_validate_layer(None) == _lib.RMOE_ENULL
    bad = _layer(bits=3)
    assert lib.rmoe_validate_layer(ctypes.byref(bad)) == _lib.RMOE_EBITS
    bad = _layer()
    bad.gate_up.group_size = 32
    assert lib.rmoe_validate_layer(ctypes.byref(bad)) == _lib.RMOE_EBITS
    bad = _layer()
    bad.gate_up.rows = 100
    assert lib.rmoe_validate_layer(ctypes.byref(bad)) == _lib.RMOE_EINVAL
    assert b"2*inter" in lib.rmoe_last_error()
    bad = _layer()
    bad.router_w = FAKE + 2
    assert lib.rmoe_validate_layer(ctypes.byref(bad)) == _lib.RMOE_EALIGN
    bad = _layer()
    bad.top_k = 5
    assert lib.rmoe_validate_layer(ctypes.byref(bad)) == _lib.RMOE_EINVAL
    bad = _layer(shared=False)
    bad.shared_gate_w = FAKE
    assert lib.rmoe_validate_layer(ctypes.byref(bad)) == _lib.RMOE_EINVAL
    bad = _layer()
    bad.down.bits = 4
    bad.down.cols = 64
    assert lib.rmoe_validate_layer(ctypes.byref(bad)) == _lib.RMOE_EBITS


def _qlayer(E=4, H=256, I=64, K=2, shared=True):
    """A layer with 8-bit quantized router and shared gate."""
    L = _layer(8, E, H, I, K, shared)
    L.router_w = None
    L.shared_gate_w = None
    L.router_q = _qw(8, 1, E, H)
    if shared:
        L.shared_gate_q = _qw(8, 1, 1, H)
    return L


def test_layer_struct_matches_the_header():
    """The Python mirror of rmoe_layer has the C layout: the quantized gates
    sit after the four banks (fields appended in ABI version 2)."""
    q = ctypes.sizeof(_lib.QWeight)
    assert q == 3 * 8 + 5 * 4 + 4          # three pointers, five int32, padding
    assert _lib.Layer.router_q.offset == _lib.Layer.gate_up.offset + 4 * q
    assert _lib.Layer.shared_gate_q.offset == _lib.Layer.router_q.offset + q
    text = (ROOT / "include" / "rmoe.h").read_text()
    body = text[text.index("typedef struct rmoe_layer"):text.index("} rmoe_layer;")]
    names = re.findall(r"(\w+);", body)
    assert names == [f[0] for f in _lib.Layer._fields_]


def test_validate_quantized_gates():
    lib = _lib.load()
    assert lib.rmoe_validate_layer(ctypes.byref(_qlayer())) == _lib.RMOE_OK
    assert lib.rmoe_validate_layer(ctypes.byref(_qlayer(shared=False))) == _lib.RMOE_OK
    both = _qlayer()
    both.router_w = FAKE
    assert lib.rmoe_validate_layer(ctypes.byref(both)) == _lib.RMOE_EINVAL
    assert b"exactly one of router_w" in lib.rmoe_last_error()
    neither = _layer()
    neither.router_w = None
    assert lib.rmoe_validate_layer(ctypes.byref(neither)) == _lib.RMOE_ENULL
    four = _qlayer()
    four.router_q.bits = 4
    four.router_q.cols = 256
    assert lib.rmoe_validate_layer(ctypes.byref(four)) == _lib.RMOE_EBITS
    assert b"must be 8-bit" in lib.rmoe_last_error()
    rows = _qlayer()
    rows.router_q.rows = 5
    assert lib.rmoe_validate_layer(ctypes.byref(rows)) == _lib.RMOE_EINVAL
    mixed = _qlayer()
    mixed.shared_gate_q = _lib.QWeight()
    mixed.shared_gate_w = FAKE
    assert lib.rmoe_validate_layer(ctypes.byref(mixed)) == _lib.RMOE_EINVAL
    assert b"router's format" in lib.rmoe_last_error()
    mixed = _layer()
    mixed.shared_gate_q = _qw(8, 1, 1, 256)
    mixed.shared_gate_w = None
    assert lib.rmoe_validate_layer(ctypes.byref(mixed)) == _lib.RMOE_EINVAL
    sg = _qlayer()
    sg.shared_gate_q.rows = 2
    assert lib.rmoe_validate_layer(ctypes.byref(sg)) == _lib.RMOE_EINVAL
    no_shared = _qlayer(shared=False)
    no_shared.shared_gate_q = _qw(8, 1, 1, 256)
    assert lib.rmoe_validate_layer(ctypes.byref(no_shared)) == _lib.RMOE_EINVAL


def test_post_norm_validation_and_rms_norm_arguments():
    lib = _lib.load()
    L = _layer()
    L.post_norm_w = FAKE
    L.norm_eps = 1e-6
    assert lib.rmoe_validate_layer(ctypes.byref(L)) == _lib.RMOE_OK
    L.post_norm_w = FAKE + 2
    assert lib.rmoe_validate_layer(ctypes.byref(L)) == _lib.RMOE_EALIGN
    L.post_norm_w = FAKE
    for bad in (-1e-6, float("nan"), 2.0):
        L.norm_eps = bad
        assert lib.rmoe_validate_layer(ctypes.byref(L)) == _lib.RMOE_EINVAL
    L.norm_eps = 1e-5
    plain = lib.rmoe_workspace_bytes(ctypes.byref(_layer()), 5)
    assert lib.rmoe_workspace_bytes(ctypes.byref(L), 5) >= plain + 5 * 256 * 2
    assert lib.rmoe_rms_norm(FAKE, FAKE, 3, 100, 1e-6, FAKE, None) == _lib.RMOE_EINVAL
    assert lib.rmoe_rms_norm(FAKE, FAKE, 3, 128, -1.0, FAKE, None) == _lib.RMOE_EINVAL
    assert lib.rmoe_rms_norm(FAKE + 2, FAKE, 3, 128, 1e-6, FAKE, None) == _lib.RMOE_EALIGN
    assert lib.rmoe_rms_norm(None, FAKE, 3, 128, 1e-6, FAKE, None) == _lib.RMOE_ENULL
    assert lib.rmoe_rms_norm(None, None, 0, 128, 1e-6, None, None) == _lib.RMOE_OK
    normed = _layer(H=2048, I=512, E=256, K=8)
    normed.post_norm_w = FAKE
    layers = (_lib.Layer * 2)(normed, _layer(H=2048, I=512, E=256, K=8))
    buf = (ctypes.c_uint8 * lib.rmoe_chain_table_bytes(2))()
    assert lib.rmoe_chain_table_pack(layers, 2, ctypes.addressof(buf)) == _lib.RMOE_EINVAL
    assert b"layer 1 differs" in lib.rmoe_last_error()


def test_quantized_router_rejects_before_launch():
    lib = _lib.load()
    r = _qw(8, 1, 16, 256)
    need = lib.rmoe_router_workspace_bytes(16, 2, 3)
    assert lib.rmoe_router_q(None, 2, 1, FAKE, 3, FAKE, FAKE, FAKE, need, None) == _lib.RMOE_ENULL
    assert lib.rmoe_router_q(ctypes.byref(r), 17, 1, FAKE, 3, FAKE, FAKE, FAKE, need,
                             None) == _lib.RMOE_EINVAL
    assert lib.rmoe_router_q(ctypes.byref(r), 2, 1, FAKE + 2, 3, FAKE, FAKE, FAKE, need,
                             None) == _lib.RMOE_EALIGN
    assert lib.rmoe_router_q(ctypes.byref(r), 2, 1, FAKE, 3, FAKE, FAKE, FAKE, need - 1,
                             None) == _lib.RMOE_EWS
    r4 = _qw(4, 1, 16, 256)
    assert lib.rmoe_router_q(ctypes.byref(r4), 2, 1, FAKE, 3, FAKE, FAKE, FAKE, need,
                             None) == _lib.RMOE_EBITS
    bank = _qw(8, 2, 16, 256)
    assert lib.rmoe_router_q(ctypes.byref(bank), 2, 1, FAKE, 3, FAKE, FAKE, FAKE, need,
                             None) == _lib.RMOE_EINVAL
    assert lib.rmoe_router_q(ctypes.byref(r), 2, 1, FAKE, 0, None, None, None, 0,
                             None) == _lib.RMOE_OK


def test_quantized_gate_prefill_workspace_holds_the_split_planes():
    """A call that takes the matrix-core router needs room for the two bf16
    planes of an 8-bit gate (2 * E * H * 2 bytes) beyond the bf16 layout."""
    lib = _lib.load()
    T = 256
    bf = lib.rmoe_workspace_bytes(ctypes.byref(_layer(E=64, H=512, I=128, K=4)), T)
    q = lib.rmoe_workspace_bytes(ctypes.byref(_qlayer(E=64, H=512, I=128, K=4)), T)
    assert q - bf >= 2 * 64 * 512 * 2
    assert lib.rmoe_workspace_bytes(ctypes.byref(_qlayer(E=64, H=512, I=128, K=4)), 1) == \
        lib.rmoe_workspace_bytes(ctypes.byref(_layer(E=64, H=512, I=128, K=4)), 1)


def test_chain_table_pack_rejects_mixed_gate_formats():
    lib = _lib.load()
    layers = (_lib.Layer * 2)(_layer(H=2048, I=512, E=256, K=8),
                              _qlayer(H=2048, I=512, E=256, K=8))
    n = lib.rmoe_chain_table_bytes(2)
    buf = (ctypes.c_uint8 * n)()
    assert lib.rmoe_chain_table_pack(layers, 2, ctypes.addressof(buf)) == _lib.RMOE_EINVAL
    assert b"layer 1 differs" in lib.rmoe_last_error()


def test_block_rejects_before_launch():
    lib = _lib.load()
    L = _layer()
    need = lib.rmoe_workspace_bytes(ctypes.byref(L), 1)
    assert need > 0
    P = ctypes.c_void_p
    # workspace too small / missing
    rc = lib.rmoe_moe_block(ctypes.byref(L), FAKE, 1, None, FAKE + 4096, None, None,
                            FAKE, need - 1, None)
    assert rc == _lib.RMOE_EWS
    rc = lib.rmoe_moe_block(ctypes.byref(L), FAKE, 1, None, FAKE + 4096, None, None,
                            None, 0, None)
    assert rc == _lib.RMOE_EWS
    # misaligned x, aliasing out, token count
    rc = lib.rmoe_moe_block(ctypes.byref(L), FAKE + 2, 1, None, FAKE, None, None, FAKE, need, None)
    assert rc == _lib.RMOE_EALIGN
    rc = lib.rmoe_moe_block(ctypes.byref(L), FAKE, 1, None, FAKE, None, None, FAKE, need, None)
    assert rc == _lib.RMOE_EINVAL
    rc = lib.rmoe_moe_block(ctypes.byref(L), FAKE, -1, None, FAKE + 64, None, None, FAKE, need, None)
    assert rc == _lib.RMOE_EINVAL
    # zero tokens is a no-op
    assert lib.rmoe_moe_block(ctypes.byref(L), FAKE, 0, None, FAKE + 64, None, None,
                              None, 0, None) == _lib.RMOE_OK
    del P


def test_switch_and_qmm_reject_before_launch():
    lib = _lib.load()
    gu, dn = _qw(8, 4, 128, 256), _qw(8, 4, 256, 64)
    need = lib.rmoe_switch_workspace_bytes(ctypes.byref(gu), ctypes.byref(dn), 2, 2)
    assert lib.rmoe_switch_glu(ctypes.byref(gu), ctypes.byref(dn), FAKE, 2, FAKE, 0, FAKE,
                               FAKE, need, None) == _lib.RMOE_EINVAL
    bad_dn = _qw(8, 4, 255, 64)
    assert lib.rmoe_switch_glu(ctypes.byref(gu), ctypes.byref(bad_dn), FAKE, 2, FAKE, 2, FAKE,
                               FAKE, need, None) == _lib.RMOE_EINVAL
    assert lib.rmoe_switch_glu(ctypes.byref(gu), ctypes.byref(dn), FAKE, 2, FAKE, 2, FAKE,
                               FAKE, need - 256, None) == _lib.RMOE_EWS
    w = _qw(8, 1, 32, 256)
    assert lib.rmoe_gather_qmm(FAKE, 1, None, None, 1, ctypes.byref(w), FAKE, FAKE,
                               None) == _lib.RMOE_EINVAL  # both outputs given
    assert lib.rmoe_gather_qmm(FAKE, 1, None, None, 1, ctypes.byref(w), None, None,
                               None) == _lib.RMOE_EINVAL
    w_odd = _qw(8, 1, 32, 192)  # 12 chunks per row: not a power of two
    assert lib.rmoe_gather_qmm(FAKE, 1, None, None, 1, ctypes.byref(w_odd), FAKE, None,
                               None) == _lib.RMOE_EINVAL


def test_switch_combine_rejects_before_launch():
    lib = _lib.load()
    gu, dn = _qw(8, 4, 256, 256), _qw(8, 4, 256, 128)
    need = lib.rmoe_switch_combine_workspace_bytes(ctypes.byref(gu), ctypes.byref(dn), 32, 2)
    assert need > lib.rmoe_switch_workspace_bytes(ctypes.byref(gu), ctypes.byref(dn), 32, 2)
    args = (ctypes.byref(gu), ctypes.byref(dn), FAKE, 32)
    assert lib.rmoe_switch_combine(*args, FAKE, None, 2, None, FAKE + 4096, FAKE, need,
                                   None) == _lib.RMOE_ENULL          # no weights
    assert lib.rmoe_switch_combine(*args, FAKE, FAKE, 2, None, FAKE, FAKE, need,
                                   None) == _lib.RMOE_EINVAL         # out aliases x
    # 64 routed rows take the sorted path: 16-byte aligned rows required
    assert lib.rmoe_switch_combine(*args, FAKE, FAKE, 2, None, FAKE + 4098, FAKE, need,
                                   None) == _lib.RMOE_EALIGN
    assert lib.rmoe_switch_combine(*args, FAKE, FAKE, 2, FAKE + 2, FAKE + 4096, FAKE, need,
                                   None) == _lib.RMOE_EALIGN
    assert lib.rmoe_switch_combine(*args, FAKE, FAKE, 2, None, FAKE + 4096, FAKE, need - 256,
                                   None) == _lib.RMOE_EWS
    assert lib.rmoe_switch_glu(*args, FAKE, 2, FAKE + 2, FAKE,
                               lib.rmoe_switch_workspace_bytes(ctypes.byref(gu),
                                                               ctypes.byref(dn), 32, 2),
                               None) == _lib.RMOE_EALIGN


def test_router_quantize_stream_reject_before_launch():
    lib = _lib.load()
    assert lib.rmoe_router(FAKE, 16, 100, 2, 1, FAKE, 1, FAKE, FAKE, FAKE, 1 << 20,
                           None) == _lib.RMOE_EINVAL  # hidden not a multiple of 64
    assert lib.rmoe_router(FAKE, 16, 128, 17, 1, FAKE, 1, FAKE, FAKE, FAKE, 1 << 20,
                           None) == _lib.RMOE_EINVAL  # top_k > experts
    assert lib.rmoe_quantize(FAKE, 4, 64, 5, 64, FAKE, FAKE, FAKE, None) == _lib.RMOE_EBITS
    assert lib.rmoe_quantize(FAKE, 4, 100, 8, 64, FAKE, FAKE, FAKE, None) == _lib.RMOE_EINVAL
    w = _qw(8, 2, 16, 128)
    assert lib.rmoe_dequantize(ctypes.byref(w), 30, 4, FAKE, None, None) == _lib.RMOE_EINVAL
    assert lib.rmoe_stream_read(FAKE, 100, FAKE, 4, None) == _lib.RMOE_EALIGN
    assert lib.rmoe_stream_read(FAKE, 4096, FAKE, 0, None) == _lib.RMOE_EINVAL


def test_chain_table_pack_rejects_mixed_layers():
    lib = _lib.load()
    layers = (_lib.Layer * 2)(_layer(), _layer(E=8))
    n = lib.rmoe_chain_table_bytes(2)
    buf = (ctypes.c_uint8 * n)()
    assert lib.rmoe_chain_table_pack(layers, 2, ctypes.addressof(buf)) == _lib.RMOE_EINVAL
    assert b"layer 1 differs" in lib.rmoe_last_error()
    assert lib.rmoe_chain_table_bytes(0) == 0


def test_status_strings():
    lib = _lib.load()
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert lib.rmoe_status_string(code)
    assert lib.rmoe_workspace_status_offset() > 0


def test_python_raises_value_error_with_the_message():
    lib = _lib.load()
    bad = _layer(bits=3)
    with pytest.raises(ValueError, match="bits must be 4 or 8"):
        _lib.check(lib.rmoe_validate_layer(ctypes.byref(bad)))


# ---------------------------------------------------------------- modules

def _switch(bits=8, E=4, H=128, I=64, device="cpu"):
    from runnel_amd import SwitchGLU
    m = SwitchGLU(H, I, E, bits=bits, device=device)
    g = torch.Generator().manual_seed(0)
    for proj in (m.gate_proj, m.up_proj, m.down_proj):
        proj.weight.copy_(torch.randint(-2**31, 2**31 - 1, proj.weight.shape, generator=g,
                                        dtype=torch.int64).to(torch.int32))
        proj.scales.copy_(torch.randn(proj.scales.shape, generator=g).to(torch.bfloat16))
        proj.biases.copy_(torch.randn(proj.biases.shape, generator=g).to(torch.bfloat16))
    return m


def test_fused_module_packs_up_then_gate():
    from runnel_amd import FusedQuantizedSwitchGLU
    old = _switch()
    fused = FusedQuantizedSwitchGLU(old)
    assert torch.equal(fused.weight, torch.cat([old.up_proj.weight, old.gate_proj.weight], 1))
    assert torch.equal(fused.scales, torch.cat([old.up_proj.scales, old.gate_proj.scales], 1))
    assert torch.equal(fused.biases, torch.cat([old.up_proj.biases, old.gate_proj.biases], 1))
    assert fused.bits == 8 and fused.group_size == 64 and fused.mode == "affine"
    assert fused.down_proj is old.down_proj and fused.activation is old.activation
    assert "weight" in fused and fused.get("bias") is None


def test_fused_module_error_messages():
    from runnel_amd import FusedQuantizedSwitchGLU
    old = _switch()
    old.gate_proj.bits = 4
    with pytest.raises(ValueError, match="^routed gate/up quantization formats differ$"):
        FusedQuantizedSwitchGLU(old)
    old = _switch()
    old.up_proj.register_buffer("bias", torch.zeros(4, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="^module biases are not expected for this checkpoint$"):
        FusedQuantizedSwitchGLU(old)
    old = _switch()
    old.gate_proj.register_buffer("biases", None)
    with pytest.raises(ValueError, match="^routed gate/up affine-bias formats differ$"):
        FusedQuantizedSwitchGLU(old)


class _Obj:
    pass


def _fake_model(n_layers, quantized=True):
    model = _Obj()
    model.language_model = _Obj()
    model.language_model.layers = []
    for _ in range(n_layers):
        layer = _Obj()
        layer.mlp = _Obj()
        layer.mlp.switch_mlp = _switch()
        if not quantized:
            del layer.mlp.switch_mlp.gate_proj.bits
        model.language_model.layers.append(layer)
    return model


def test_fuse_routed_gate_up_counts_and_replaces():
    from runnel_amd import FusedQuantizedSwitchGLU, fuse_routed_gate_up
    model = _fake_model(3)
    assert fuse_routed_gate_up(model) == 3
    for layer in model.language_model.layers:
        assert isinstance(layer.mlp.switch_mlp, FusedQuantizedSwitchGLU)


def test_fuse_routed_gate_up_requires_quantized_projections():
    from runnel_amd import fuse_routed_gate_up
    model = _fake_model(1, quantized=False)
    with pytest.raises(ValueError, match="^routed gate/up are not quantized as expected$"):
        fuse_routed_gate_up(model)


def test_kernels_refuse_host_tensors():
    from runnel_amd import native
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    w = torch.zeros(1, 32, 32, dtype=torch.int32)
    s = torch.zeros(1, 32, 2, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensors"):
        native.gather_qmm(x, w, s, s, 8)
    with pytest.raises(ValueError, match="GPU tensors"):
        native.quantize(torch.zeros(4, 64), 8)


def test_bench_byte_model_matches_the_layer_byte_counts():
    import bench
    assert bench.layer_bytes(2048, 512, 256, 8, 8) == 31_141_888
    assert bench.layer_bytes(2048, 512, 256, 8, 4) == 16_986_112
    # 8-bit gates: 256 rows of 2048 codes + 32 (scale, bias) pairs, and one
    # such row for the shared gate, instead of 257 bf16 rows
    q = bench.layer_bytes(2048, 512, 256, 8, 8, gate_bits=8)
    assert 31_141_888 - q == 257 * (4096 - (2048 + 128))


def test_cooperative_launch_switch_returns_previous_mode():
    """rmoe_set_cooperative_launch is process-wide and returns the previous
    mode; plain launches are the default."""
    lib = _lib.load()
    assert lib.rmoe_set_cooperative_launch(1) == 0
    assert lib.rmoe_set_cooperative_launch(0) == 1
    assert lib.rmoe_set_cooperative_launch(7) == 0   # any nonzero turns it on
    assert lib.rmoe_set_cooperative_launch(0) == 1


def test_single_launch_shape_rejects_nine_routed_slots():
    """The single-launch kernel ranks at most 8 routed slots: a top-9 layer
    without a shared expert is refused by the chained decode on the host
    (the shape check needs no device), and a one-token block call of it takes
    the multi-kernel path instead."""
    lib = _lib.load()
    n = lib.rmoe_chain_table_bytes(1)
    buf = (ctypes.c_uint8 * n)()
    top9 = (_lib.Layer * 1)(_layer(H=2048, I=512, E=16, K=9, shared=False))
    assert lib.rmoe_validate_layer(top9) == _lib.RMOE_OK
    assert lib.rmoe_chain_table_pack(top9, 1, ctypes.addressof(buf)) == _lib.RMOE_EINVAL
    assert b"top_k <= 8" in lib.rmoe_last_error()
    big = (_lib.Layer * 1)(_layer(H=2048, I=512, E=257, K=8))
    assert lib.rmoe_chain_table_pack(big, 1, ctypes.addressof(buf)) == _lib.RMOE_EINVAL
    assert b"experts <= 256" in lib.rmoe_last_error()


def test_hidden_limit_of_the_few_token_gate_up_kernel():
    """The few-token gate/up kernel covers 256 16-byte chunks per row:
    hidden <= 4096 at 8 bits and <= 8192 at 4 bits; wider layers are refused
    before anything is launched rather than silently truncated."""
    lib = _lib.load()
    for bits, ok_h in ((8, 4096), (4, 8192)):
        assert lib.rmoe_validate_layer(ctypes.byref(_layer(bits=bits, H=ok_h))) == _lib.RMOE_OK
        rc = lib.rmoe_validate_layer(ctypes.byref(_layer(bits=bits, H=ok_h + 64)))
        assert rc == _lib.RMOE_EINVAL
        assert b"too large" in lib.rmoe_last_error()
    gu, dn = _qw(8, 4, 128, 4160), _qw(8, 4, 4160, 64)
    need = lib.rmoe_switch_workspace_bytes(ctypes.byref(gu), ctypes.byref(dn), 2, 2)
    assert lib.rmoe_switch_glu(ctypes.byref(gu), ctypes.byref(dn), FAKE, 2, FAKE, 2, FAKE,
                               FAKE, need, None) == _lib.RMOE_EINVAL


def _host_handle(H=256):
    from runnel_amd import native
    return native.LayerHandle(_layer(H=H), ())


def test_python_block_checks_shapes_before_the_library():
    """x, residual and out are checked against [tokens, hidden] (and out for
    dtype and contiguity) before any pointer is handed over: the library
    trusts the shapes it is given."""
    from runnel_amd import native
    h = _host_handle(256)
    bf = torch.bfloat16
    with pytest.raises(ValueError, match=r"x must be \[tokens, 256\]"):
        native.moe_block(h, torch.zeros(2, 128, dtype=bf))
    with pytest.raises(ValueError, match="x must be a 2-D bfloat16"):
        native.moe_block(h, torch.zeros(2, 256, dtype=torch.float32))
    x = torch.zeros(2, 256, dtype=bf)
    with pytest.raises(ValueError, match=r"residual must be \[2, 256\]"):
        native.moe_block(h, x, residual=torch.zeros(2, 128, dtype=bf))
    with pytest.raises(ValueError, match="residual must be bfloat16"):
        native.moe_block(h, x, residual=torch.zeros(2, 256))
    with pytest.raises(ValueError, match="out must be bfloat16"):
        native.moe_block(h, x, out=torch.zeros(2, 256, dtype=torch.float16))
    with pytest.raises(ValueError, match=r"out must be \[2, 256\]"):
        native.moe_block(h, x, out=torch.zeros(1, 256, dtype=bf))
    with pytest.raises(ValueError, match="out must be contiguous"):
        native.moe_block(h, x, out=torch.zeros(256, 2, dtype=bf).t())
    # well-formed host tensors get as far as the device check
    with pytest.raises(ValueError, match="GPU tensors"):
        native.moe_block(h, x, residual=torch.zeros(4, 256, dtype=bf)[::2])


def test_python_switch_and_qmm_check_shapes_before_the_library():
    from runnel_amd import native
    bf = torch.bfloat16
    gu, dn = _qw(8, 4, 128, 256), _qw(8, 4, 256, 64)
    idx = torch.zeros(2, 2, dtype=torch.int32)
    with pytest.raises(ValueError, match=r"x must be \[2, 256\]"):
        native.switch_glu(torch.zeros(2, 128, dtype=bf), idx, gu, dn)
    with pytest.raises(ValueError, match=r"x must be \[2, 256\]"):
        native.switch_combine(torch.zeros(3, 256, dtype=bf), idx, torch.zeros(2, 2), gu, dn)
    with pytest.raises(ValueError, match=r"weights must be \[2, 2\]"):
        native.switch_combine(torch.zeros(2, 256, dtype=bf), idx, torch.zeros(2, 3), gu, dn)
    with pytest.raises(ValueError, match=r"residual must be \[2, 256\]"):
        native.switch_combine(torch.zeros(2, 256, dtype=bf), idx, torch.zeros(2, 2), gu, dn,
                              residual=torch.zeros(2, 255, dtype=bf))
    w = torch.zeros(1, 32, 32, dtype=torch.int32)   # 128 columns at 8 bits
    s = torch.zeros(1, 32, 2, dtype=bf)
    with pytest.raises(ValueError, match="x has 256 columns, the weight 128"):
        native.gather_qmm(torch.zeros(1, 256, dtype=bf), w, s, s, 8)


def test_layer_weights_must_live_on_the_gpu():
    from runnel_amd import native
    bf = torch.bfloat16
    bank = (torch.zeros(4, 128, 64, dtype=torch.int32), torch.zeros(4, 128, 4, dtype=bf),
            torch.zeros(4, 128, 4, dtype=bf))
    dbank = (torch.zeros(4, 256, 16, dtype=torch.int32), torch.zeros(4, 256, 1, dtype=bf),
             torch.zeros(4, 256, 1, dtype=bf))
    with pytest.raises(ValueError, match="GPU tensors"):
        native.make_layer(torch.zeros(4, 256, dtype=bf), bank, dbank, 2)
    with pytest.raises(ValueError, match="GPU tensors"):
        native.qweight_struct(*bank, 8)


def test_status_word_is_read_cleared_and_raised():
    """check_status raises RmoeError(RMOE_ETIMEOUT) once for a set (sticky)
    status word and clears it; workspace_status reads it without clearing
    unless asked."""
    from runnel_amd import native
    lib = _lib.load()
    off = lib.rmoe_workspace_status_offset()
    ws = torch.zeros(off + 256, dtype=torch.uint8)
    native.check_status(ws)                       # clear: nothing raised
    ws[off:off + 4].view(torch.int32).fill_(1)
    assert native.workspace_status(ws) == 1
    assert native.workspace_status(ws) == 1       # reading does not clear
    with pytest.raises(_lib.RmoeError) as e:
        native.check_status(ws)
    assert e.value.status == _lib.RMOE_ETIMEOUT
    assert native.workspace_status(ws) == 0
    native.check_status(ws)
    assert b"timed out" in lib.rmoe_status_string(_lib.RMOE_ETIMEOUT)


def test_noalloc_block_refuses_calls_beyond_its_static_scratch():
    """rmoe_moe_block_noalloc checks the call's scratch need against its
    fixed static array before it touches the device."""
    lib = _lib.load()
    L = _layer(H=2048, I=512, E=256, K=8)
    T = 1
    while lib.rmoe_workspace_bytes(ctypes.byref(L), T) <= _lib.NOALLOC_SCRATCH_BYTES:
        T *= 2
    rc = lib.rmoe_moe_block_noalloc(ctypes.byref(L), FAKE, T, None, FAKE + (1 << 24), None,
                                    None, None, None)
    assert rc == _lib.RMOE_EWS
    assert b"static scratch" in lib.rmoe_last_error()
    # argument errors come first, and zero tokens is a no-op
    assert lib.rmoe_moe_block_noalloc(ctypes.byref(L), FAKE, 1, None, FAKE, None, None, None,
                                      None) == _lib.RMOE_EINVAL   # out aliases x
    assert lib.rmoe_moe_block_noalloc(ctypes.byref(L), FAKE, 1, None, FAKE + 4096, None, None,
                                      FAKE + 2, None) == _lib.RMOE_EALIGN
    assert lib.rmoe_moe_block_noalloc(ctypes.byref(L), FAKE, 0, None, FAKE + 4096, None, None,
                                      None, None) == _lib.RMOE_OK
