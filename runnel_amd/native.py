"""torch-facing wrappers over the C ABI (include/rmoe.h).

Every function here hands device pointers of torch tensors to librmoe.so
and enqueues the HIP kernels on torch's current stream; nothing computes on
the host.  Packed weights are carried as int32 tensors (the same bits as
MLX's uint32 words); scales, biases and activations as bfloat16.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib

BF16 = torch.bfloat16


def _require_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("runnel_amd kernels take GPU tensors")


def _check_rows(t: torch.Tensor, name: str, rows: int, cols: int) -> None:
    """t must be a bf16 [rows, cols] tensor (checked before any pointer
    reaches the library, which trusts the shapes it is given)."""
    if t.dtype != BF16:
        raise ValueError(f"{name} must be bfloat16 (got {t.dtype})")
    if t.dim() != 2 or tuple(t.shape) != (rows, cols):
        raise ValueError(f"{name} must be [{rows}, {cols}] (got {list(t.shape)})")


def _check_out(out: torch.Tensor, rows: int, cols: int) -> None:
    _check_rows(out, "out", rows, cols)
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")


def _check_x(x: torch.Tensor, cols: int) -> None:
    if x.dtype != BF16 or x.dim() != 2:
        raise ValueError("x must be a 2-D bfloat16 tensor")
    if x.shape[1] != cols:
        raise ValueError(f"x must be [tokens, {cols}] (got {list(x.shape)})")


def values_per_word(bits: int) -> int:
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8 (got {bits})")
    return 32 // bits


def qweight_struct(weight, scales, biases, bits: int, group_size: int = 64) -> _lib.QWeight:
    """rmoe_qweight for a bank [E, rows, K*bits/32] (or a matrix without the
    expert axis)."""
    if weight.dim() == 2:
        experts, rows, words = 1, weight.shape[0], weight.shape[1]
    elif weight.dim() == 3:
        experts, rows, words = weight.shape
    else:
        raise ValueError("packed weight must be 2-D or 3-D")
    for t, name in ((weight, "weight"), (scales, "scales"), (biases, "biases")):
        if t is None:
            raise ValueError(f"{name} is required")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    _require_cuda(weight, scales, biases)
    if weight.dtype not in (torch.int32, getattr(torch, "uint32", torch.int32)):
        raise ValueError("packed weight must be int32/uint32")
    if scales.dtype != BF16 or biases.dtype != BF16:
        raise ValueError("scales and biases must be bfloat16")
    cols = words * values_per_word(bits)
    return _lib.QWeight(weight.data_ptr(), scales.data_ptr(), biases.data_ptr(),
                        experts, rows, cols, bits, group_size)


class Workspace:
    """Grow-only, zero-initialised device scratch per (device, stream,
    purpose).  The library keeps its counters at zero between calls, so the
    buffer is zeroed only when it is (re)allocated.  Calls on one stream run
    in order and may share a buffer; calls on different streams may overlap,
    so each stream gets its own (the library's calls are safe concurrently
    on different streams only with different workspaces)."""

    def __init__(self):
        self._bufs: dict = {}

    @staticmethod
    def _key(device, key: str):
        d = torch.device(device)
        if d.index is None:
            d = torch.device(d.type, torch.cuda.current_device())
        return (str(d), torch.cuda.current_stream(d).cuda_stream, key)

    def peek(self, device, key: str = "default") -> torch.Tensor | None:
        return self._bufs.get(self._key(device, key))

    def get(self, device, nbytes: int, key: str = "default") -> torch.Tensor:
        k = self._key(device, key)
        buf = self._bufs.get(k)
        if buf is None or buf.numel() < nbytes:
            # 256-byte alignment comes from the caching allocator (512 B).
            buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
            self._bufs[k] = buf
        return buf


WORKSPACE = Workspace()


def gather_qmm(x: torch.Tensor, weight, scales, biases, bits: int, group_size: int = 64,
               rhs_indices: torch.Tensor | None = None,
               lhs_indices: torch.Tensor | None = None,
               out_dtype=BF16) -> torch.Tensor:
    """y[m] = x[lhs[m]] @ dequantize(weight[rhs[m]]).T  (mx.gather_qmm with
    transpose=True, called at src/runnel/mlx.py:64-75).

    x: bf16 [x_rows, K]; rhs_indices / lhs_indices: int32 [M] (None: expert
    0 / row m).  Returns [M, N] in bf16 or float32."""
    lib = _lib.load()
    if x.dtype != BF16 or x.dim() != 2:
        raise ValueError("x must be a 2-D bfloat16 tensor")
    cols = weight.shape[-1] * values_per_word(bits)
    if x.shape[1] != cols:
        raise ValueError(f"x has {x.shape[1]} columns, the weight {cols}")
    _require_cuda(x, weight, rhs_indices, lhs_indices)
    x = x.contiguous()
    qw = qweight_struct(weight, scales, biases, bits, group_size)
    if lhs_indices is not None:
        lhs_indices = lhs_indices.to(torch.int32).contiguous()
        M = lhs_indices.numel()
    elif rhs_indices is not None:
        M = rhs_indices.numel()
    else:
        M = x.shape[0]
    if rhs_indices is not None:
        rhs_indices = rhs_indices.to(torch.int32).contiguous()
        if rhs_indices.numel() != M:
            raise ValueError("rhs_indices must have one entry per output row")
    if lhs_indices is None and x.shape[0] != M:
        raise ValueError("x must have one row per output row when lhs_indices is None")
    y = torch.empty((M, qw.rows), dtype=out_dtype, device=x.device)
    if out_dtype not in (BF16, torch.float32):
        raise ValueError("out_dtype must be bfloat16 or float32")
    _lib.check(lib.rmoe_gather_qmm(
        x.data_ptr(), x.shape[0], _lib.ptr(lhs_indices), _lib.ptr(rhs_indices), M,
        ctypes.byref(qw), y.data_ptr() if out_dtype == BF16 else None,
        y.data_ptr() if out_dtype == torch.float32 else None,
        _lib.stream_handle(x.device)))
    return y


def switch_glu(x: torch.Tensor, indices: torch.Tensor, gate_up: _lib.QWeight,
               down: _lib.QWeight) -> torch.Tensor:
    """Packed [up; gate] projection + SwiGLU + down per (token, slot):
    x bf16 [T, H], indices int [T, k] -> bf16 [T, k, H] (uncombined)."""
    lib = _lib.load()
    if indices.dim() != 2:
        raise ValueError("indices must be [tokens, k]")
    T, k = indices.shape
    H = gate_up.cols
    _check_rows(x, "x", T, H)
    _require_cuda(x, indices)
    x = x.contiguous()
    idx = indices.to(torch.int32).contiguous()
    y = torch.empty((T, k, H), dtype=BF16, device=x.device)
    need = lib.rmoe_switch_workspace_bytes(ctypes.byref(gate_up), ctypes.byref(down), T, k)
    ws = WORKSPACE.get(x.device, need, "switch")
    _lib.check(lib.rmoe_switch_glu(ctypes.byref(gate_up), ctypes.byref(down),
                                   x.data_ptr(), T, idx.data_ptr(), k, y.data_ptr(),
                                   ws.data_ptr(), ws.numel(),
                                   _lib.stream_handle(x.device)))
    return y


def switch_combine(x: torch.Tensor, indices: torch.Tensor, weights: torch.Tensor,
                   gate_up: _lib.QWeight, down: _lib.QWeight,
                   residual: torch.Tensor | None = None) -> torch.Tensor:
    """The routed half of the block for a given routing: x bf16 [T, H],
    indices int [T, k], weights float32 [T, k] -> bf16 [T, H] =
    bf16(sum_j weights[t, j] * y[t, j]) (+ residual)."""
    lib = _lib.load()
    if indices.dim() != 2:
        raise ValueError("indices must be [tokens, k]")
    T, k = indices.shape
    H = gate_up.cols
    _check_rows(x, "x", T, H)
    if tuple(weights.shape) != (T, k):
        raise ValueError(f"weights must be [{T}, {k}] (got {list(weights.shape)})")
    if residual is not None:
        _check_rows(residual, "residual", T, H)
    _require_cuda(x, indices, weights, residual)
    x = x.contiguous()
    idx = indices.to(torch.int32).contiguous()
    w = weights.to(torch.float32).contiguous()
    out = torch.empty((T, H), dtype=BF16, device=x.device)
    res = None if residual is None else residual.contiguous()
    need = lib.rmoe_switch_combine_workspace_bytes(ctypes.byref(gate_up), ctypes.byref(down),
                                                   T, k)
    ws = WORKSPACE.get(x.device, need, "switch")
    _lib.check(lib.rmoe_switch_combine(ctypes.byref(gate_up), ctypes.byref(down),
                                       x.data_ptr(), T, idx.data_ptr(), w.data_ptr(), k,
                                       _lib.ptr(res), out.data_ptr(), ws.data_ptr(),
                                       ws.numel(), _lib.stream_handle(x.device)))
    return out


@dataclass
class LayerHandle:
    """An rmoe_layer struct plus the tensors it points at (kept alive)."""
    struct: _lib.Layer
    tensors: tuple

    @property
    def hidden(self):
        return self.struct.hidden

    @property
    def top_k(self):
        return self.struct.top_k

    def workspace_bytes(self, tokens: int) -> int:
        return _lib.load().rmoe_workspace_bytes(ctypes.byref(self.struct), tokens)

    def validate(self):
        _lib.check(_lib.load().rmoe_validate_layer(ctypes.byref(self.struct)))


def _gate(g, rows: int | None, name: str):
    """A router / shared gate: a bf16 tensor, or a (weight, scales, biases)
    triple of an 8-bit group-64 quantized gate -> (bf16 tensor or None,
    rmoe_qweight, tensors to keep alive)."""
    if isinstance(g, (tuple, list)):
        w, s, b = (t.reshape(-1, t.shape[-1]).contiguous() for t in g)
        if rows is not None and w.shape[0] != rows:
            raise ValueError(f"{name} must have {rows} rows (got {w.shape[0]})")
        return None, qweight_struct(w, s, b, 8, 64), (w, s, b)
    return g, _lib.QWeight(), ()


def make_layer(router_w, gate_up, down, top_k: int, norm_topk_prob: bool = True,
               shared_gate_w=None, shared_gate_up=None, shared_down=None,
               bits: int = 8, group_size: int = 64, post_norm_w=None,
               norm_eps: float = 1e-6) -> LayerHandle:
    """router_w bf16 [E, H], or the (weight, scales, biases) triple of an
    8-bit group-64 quantized gate (QuantizedLinear); shared_gate_w likewise
    (bf16 [H] or a one-row triple, in the router's format); gate_up / down /
    shared_* are (weight, scales, biases) triples of packed banks; shared
    banks may omit the expert axis.  post_norm_w (bf16 [H]) puts the
    decoder's post-attention RMSNorm in front of the block."""
    gu = qweight_struct(*gate_up, bits, group_size)
    dn = qweight_struct(*down, bits, group_size)
    router_w, rq, rkeep = _gate(router_w, None, "router gate")
    keep = [*rkeep, *gate_up, *down]
    if shared_gate_up is not None:
        sgu = qweight_struct(*shared_gate_up, bits, group_size)
        sdn = qweight_struct(*shared_down, bits, group_size)
        keep += [*shared_gate_up, *shared_down]
        shared_inter = sgu.rows // 2
    else:
        sgu = _lib.QWeight()
        sdn = _lib.QWeight()
        shared_inter = 0
    sgq = _lib.QWeight()
    if shared_gate_w is not None:
        shared_gate_w, sgq, skeep = _gate(shared_gate_w, 1, "shared gate")
        keep += list(skeep)
        if shared_gate_w is not None:
            shared_gate_w = shared_gate_w.reshape(-1).contiguous()
            keep.append(shared_gate_w)
    if router_w is not None:
        if (router_w.dtype != BF16 or not router_w.is_contiguous()
                or router_w.dim() != 2):
            raise ValueError("router weight must be contiguous bfloat16 [experts, hidden]")
        keep.append(router_w)
        E, H = router_w.shape
    else:
        E, H = rq.rows, rq.cols
    if shared_gate_w is not None and (shared_gate_w.dtype != BF16
                                      or shared_gate_w.numel() != H):
        raise ValueError(f"shared gate must be bfloat16 [{H}]")
    if post_norm_w is not None:
        post_norm_w = post_norm_w.reshape(-1).contiguous()
        if post_norm_w.dtype != BF16 or post_norm_w.numel() != H:
            raise ValueError(f"post_norm_w must be bfloat16 [{H}]")
        keep.append(post_norm_w)
    _require_cuda(router_w, shared_gate_w, post_norm_w)
    s = _lib.Layer(H, gu.rows // 2, shared_inter, E, top_k, int(bool(norm_topk_prob)),
                   _lib.ptr(router_w), _lib.ptr(shared_gate_w), gu, dn, sgu, sdn, rq, sgq,
                   _lib.ptr(post_norm_w), float(norm_eps))
    h = LayerHandle(s, tuple(keep))
    h.validate()
    return h


def moe_block(layer: LayerHandle, x: torch.Tensor, residual: torch.Tensor | None = None,
              out: torch.Tensor | None = None, return_routing: bool = False,
              workspace: torch.Tensor | None = None, check: bool | None = None):
    """Whole SparseMoeBlock on x bf16 [T, H] -> bf16 [T, H].

    ``check``: True reads (and clears) the workspace's status word after the
    call and raises RmoeError (RMOE_ETIMEOUT / RMOE_EPLACEMENT) if a bounded
    wait of the call gave up (the single-launch decode, the few-token
    router); this synchronises the stream.  None (the default) checks eager
    calls below the expert-sorted threshold (T * top_k < 64) without
    waiting for the device: behind the first call on a workspace and every
    32nd after it, the word is copied to pinned host memory, and a later
    eager call on the workspace examines the copy once it has landed and
    raises then.  False skips the check; graph users call ``check_status``
    on the workspace after a replay."""
    lib = _lib.load()
    H = layer.hidden
    _check_x(x, H)
    T = x.shape[0]
    if residual is not None:
        _check_rows(residual, "residual", T, H)
    if out is not None:
        _check_out(out, T, H)
    _require_cuda(x, residual, out)
    x = x.contiguous()
    if residual is not None:
        residual = residual.contiguous()
    if out is None:
        out = torch.empty_like(x)
    idx = scores = None
    if return_routing:
        idx = torch.empty((T, layer.top_k), dtype=torch.int32, device=x.device)
        scores = torch.empty((T, layer.top_k), dtype=torch.float32, device=x.device)
    need = layer.workspace_bytes(T)
    ws = workspace if workspace is not None else WORKSPACE.get(x.device, need, "block")
    deferred = check is None and T * layer.top_k < _SORTED_ROWS and not _capturing(x.device)
    if deferred:
        _STATUS.poll(ws)
    _lib.check(lib.rmoe_moe_block(ctypes.byref(layer.struct), x.data_ptr(), T,
                                  _lib.ptr(residual), out.data_ptr(), _lib.ptr(idx),
                                  _lib.ptr(scores), ws.data_ptr(), ws.numel(),
                                  _lib.stream_handle(x.device)))
    if check:
        check_status(ws)
    elif deferred:
        _STATUS.after_call(ws)
    if return_routing:
        return out, idx, scores
    return out


class Chain:
    """A stack of layers for the single-launch chained decode
    (rmoe_moe_chain): x_{l+1} = bf16(x_l + block_l(x_l))."""

    def __init__(self, layers: list[LayerHandle], device="cuda"):
        lib = _lib.load()
        n = len(layers)
        if n < 1:
            raise ValueError("a chain needs at least one layer")
        arr = (_lib.Layer * n)(*[h.struct for h in layers])
        nbytes = lib.rmoe_chain_table_bytes(n)
        host = (ctypes.c_uint8 * nbytes)()
        _lib.check(lib.rmoe_chain_table_pack(arr, n, ctypes.addressof(host)))
        self.table = torch.frombuffer(bytearray(host), dtype=torch.uint8).to(device)
        self.layers = layers
        self.n = n

    def workspace_bytes(self) -> int:
        return self.layers[0].workspace_bytes(1)


def moe_chain(chain: Chain, x: torch.Tensor, out: torch.Tensor | None = None,
              workspace: torch.Tensor | None = None,
              check: bool | None = None) -> torch.Tensor:
    """One token x bf16 [1, H] (or [H]) through every layer of the chain.
    ``check`` as for ``moe_block`` (None: the deferred check of eager
    calls)."""
    lib = _lib.load()
    H = chain.layers[0].hidden
    if x.dtype != BF16 or x.numel() != H or x.dim() not in (1, 2):
        raise ValueError(f"x must be bfloat16 [1, {H}] or [{H}] (got {list(x.shape)})")
    if out is not None and (out.dtype != BF16 or out.shape != x.shape
                            or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous bfloat16 tensor of shape {list(x.shape)}")
    _require_cuda(x, out)
    x = x.contiguous()
    if out is None:
        out = torch.empty_like(x)
    ws = workspace if workspace is not None else WORKSPACE.get(
        x.device, chain.workspace_bytes(), "block")
    deferred = check is None and not _capturing(x.device)
    if deferred:
        _STATUS.poll(ws)
    _lib.check(lib.rmoe_moe_chain(ctypes.byref(chain.layers[0].struct), chain.table.data_ptr(),
                                  chain.n, x.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                  ws.numel(), _lib.stream_handle(x.device)))
    if check:
        check_status(ws)
    elif deferred:
        _STATUS.after_call(ws)
    return out


# The launch mode last set through set_cooperative_launch (the library's
# default is a plain launch).
_COOPERATIVE = [False]
# (token, slot) rows from which a block call takes the expert-sorted path,
# whose kernels do not wait on each other (src/runnel/mlx.py:59)
_SORTED_ROWS = 64


def _capturing(device) -> bool:
    return torch.cuda.is_current_stream_capturing()


def set_cooperative_launch(enabled: bool) -> bool:
    """Launch mode of the single-launch decode kernel outside graph capture
    (process-wide; returns the previous mode).  False (the library's
    default): plain launches, as a captured graph makes them (about 14 us
    per eager one-token call back to back).  True: cooperative launches,
    which guarantee that every workgroup is resident whatever runs on other
    streams, at about 18 us more per call (two plain single-launch calls
    overlapping on different streams can hold each other's CUs; their
    waits then give up and set the status word, which the deferred check
    of eager calls reports)."""
    prev = bool(_lib.load().rmoe_set_cooperative_launch(1 if enabled else 0))
    _COOPERATIVE[0] = bool(enabled)
    return prev


def workspace_status(ws: torch.Tensor, clear: bool = False) -> int:
    """The status word of a workspace: 0, or (the call's outputs are not
    valid) 1 when a single-launch decode gave up a cross-workgroup wait or
    was cancelled, 2 when a workgroup read an XCC id outside 0-7.  The word
    is sticky: every later call leaves it set until it is cleared.  Reading
    it synchronises with the work queued on ws's device."""
    off = _lib.load().rmoe_workspace_status_offset()
    word = ws[off:off + 4].view(torch.int32)
    v = int(word.item())
    if clear and v:
        word.zero_()
    return v


def _raise_status(v: int) -> None:
    if v == 2:
        raise _lib.RmoeError(_lib.RMOE_EPLACEMENT,
                             "a single-launch decode read an XCC id outside 0-7; "
                             "its outputs are not valid")
    raise _lib.RmoeError(_lib.RMOE_ETIMEOUT,
                         "a single-launch decode timed out waiting for another "
                         "workgroup; its outputs are not valid")


def check_status(ws: torch.Tensor) -> None:
    """Raise RmoeError (RMOE_ETIMEOUT, RMOE_EPLACEMENT) if the workspace's
    status word is set, clearing it first (graph users call this after a
    replay)."""
    _STATUS.forget(ws)
    v = workspace_status(ws, clear=True)
    if v:
        _raise_status(v)


class _StatusWatch:
    """The deferred check of eager single-launch calls.  Behind the first
    call on a workspace and then every `every`-th one, the status word is
    copied (4 bytes) into pinned host memory and an event recorded; the
    copy is read once that event has completed, at a later eager call on
    the workspace, so the host never waits for the device.  The word is
    sticky, so a copy also shows a failure of any call before it.  (A copy
    behind every call costs about 11 us of host time per call.)"""

    def __init__(self, every: int = 32):
        self.every = every
        self._ent: dict = {}

    def after_call(self, ws: torch.Tensor) -> None:
        key = (ws.device, ws.data_ptr())
        ent = self._ent.get(key)
        if ent is None:
            ent = [torch.zeros(1, dtype=torch.int32, pin_memory=True),
                   torch.cuda.Event(), False, 0]
            self._ent[key] = ent
        ent[3] += 1
        if ent[2] or (ent[3] - 1) % self.every:
            return
        off = _lib.load().rmoe_workspace_status_offset()
        ent[0].copy_(ws[off:off + 4].view(torch.int32), non_blocking=True)
        ent[1].record()
        ent[2] = True

    def poll(self, ws: torch.Tensor) -> None:
        ent = self._ent.get((ws.device, ws.data_ptr()))
        if ent is None or not ent[2] or not ent[1].query():
            return
        ent[2] = False
        if int(ent[0][0]):
            check_status(ws)

    def forget(self, ws: torch.Tensor) -> None:
        ent = self._ent.get((ws.device, ws.data_ptr()))
        if ent is not None:
            ent[2] = False
            ent[3] = 0


_STATUS = _StatusWatch()


def default_workspace(device, key: str = "block") -> torch.Tensor | None:
    """The library-managed workspace that calls without an explicit
    workspace use on `device` and the current stream (None before the
    first such call)."""
    return WORKSPACE.peek(device, key)


def router(router_w, x: torch.Tensor, top_k: int, norm_topk_prob: bool = True):
    """Router of the block: x bf16 [T, H], router_w bf16 [E, H] or the
    (weight, scales, biases) triple of an 8-bit group-64 quantized gate ->
    (indices int32 [T, k] in rank order, scores float32 [T, k])."""
    lib = _lib.load()
    if x.dtype != BF16 or x.dim() != 2:
        raise ValueError("x must be a 2-D bfloat16 tensor")
    T, H = x.shape
    w, rq, keep = _gate(router_w, None, "router gate")
    if w is not None and (w.dim() != 2 or w.shape[1] != H):
        raise ValueError(f"router gate must be [experts, {H}] (got {list(w.shape)})")
    _require_cuda(x, w, *keep)
    x = x.contiguous()
    E = rq.rows if w is None else w.shape[0]
    idx = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
    scores = torch.empty((T, top_k), dtype=torch.float32, device=x.device)
    need = lib.rmoe_router_workspace_bytes(E, top_k, T)
    ws = WORKSPACE.get(x.device, need, "router")
    if w is None:
        if rq.cols != H:
            raise ValueError(f"router gate has {rq.cols} columns, x has {H}")
        _lib.check(lib.rmoe_router_q(ctypes.byref(rq), top_k, int(bool(norm_topk_prob)),
                                     x.data_ptr(), T, idx.data_ptr(), scores.data_ptr(),
                                     ws.data_ptr(), ws.numel(), _lib.stream_handle(x.device)))
    else:
        w = w.contiguous()
        _lib.check(lib.rmoe_router(w.data_ptr(), E, H, top_k, int(bool(norm_topk_prob)),
                                   x.data_ptr(), T, idx.data_ptr(), scores.data_ptr(),
                                   ws.data_ptr(), ws.numel(), _lib.stream_handle(x.device)))
    return idx, scores


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm of the rows of x bf16 [..., H] with weight bf16 [H]
    (mx.fast.rms_norm) -> bf16, in the library's fixed order."""
    lib = _lib.load()
    _require_cuda(x, weight)
    if x.dtype != BF16 or weight.dtype != BF16:
        raise ValueError("rms_norm takes bfloat16 x and weight")
    H = x.shape[-1]
    x2 = x.reshape(-1, H).contiguous()
    w = weight.reshape(-1).contiguous()
    if w.numel() != H:
        raise ValueError(f"weight must have {H} values (got {w.numel()})")
    out = torch.empty_like(x2)
    _lib.check(lib.rmoe_rms_norm(x2.data_ptr(), w.data_ptr(), x2.shape[0], H, float(eps),
                                 out.data_ptr(), _lib.stream_handle(x.device)))
    return out.reshape(x.shape)


def quantize(w: torch.Tensor, bits: int, group_size: int = 64):
    """Affine quantization of float32 [..., K] on the GPU ->
    (int32 words [..., K*bits/32], bf16 scales, bf16 biases)."""
    lib = _lib.load()
    _require_cuda(w)
    if w.dtype != torch.float32:
        raise ValueError("quantize takes float32 weights")
    w = w.contiguous()
    K = w.shape[-1]
    lead = w.shape[:-1]
    rows = w.numel() // K
    wq = torch.empty((*lead, K // values_per_word(bits)), dtype=torch.int32, device=w.device)
    s = torch.empty((*lead, K // group_size), dtype=BF16, device=w.device)
    b = torch.empty_like(s)
    _lib.check(lib.rmoe_quantize(w.data_ptr(), rows, K, bits, group_size, wq.data_ptr(),
                                 s.data_ptr(), b.data_ptr(), _lib.stream_handle(w.device)))
    return wq, s, b


def dequantize(weight, scales, biases, bits: int, group_size: int = 64,
               out_dtype=torch.float32) -> torch.Tensor:
    """fl32(q*s + b) for every element ([..., K]); bf16 output rounds that
    value to nearest-even."""
    lib = _lib.load()
    _require_cuda(weight)
    qw = qweight_struct(weight, scales, biases, bits, group_size)
    rows = qw.experts * qw.rows
    out = torch.empty((*weight.shape[:-1], qw.cols), dtype=out_dtype, device=weight.device)
    _lib.check(lib.rmoe_dequantize(
        ctypes.byref(qw), 0, rows,
        out.data_ptr() if out_dtype == torch.float32 else None,
        out.data_ptr() if out_dtype == BF16 else None,
        _lib.stream_handle(weight.device)))
    return out


def stream_read(buf: torch.Tensor, blocks: int, partials: torch.Tensor | None = None):
    lib = _lib.load()
    nbytes = buf.numel() * buf.element_size()
    if partials is None:
        partials = torch.empty(blocks, dtype=torch.int32, device=buf.device)
    _lib.check(lib.rmoe_stream_read(buf.data_ptr(), nbytes, partials.data_ptr(), blocks,
                                    _lib.stream_handle(buf.device)))
    return partials
