"""Run by tests/test_zz_no_alloc.py in a fresh process: the process's first
rmoe_moe_block_noalloc calls are made under HIP graph capture (the static
scratch's address and the launch shape are resolved then), for one token
(the single-launch decode kernel) and 40 tokens (the expert-sorted path).
The graph is replayed twice with eager work between, and every replay's
outputs, indices, scores and status equal rmoe_moe_block's with a caller
workspace.  Prints "noalloc capture ok" on success."""

import ctypes
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def main():
    import torch
    from runnel_amd import _lib, native, synthetic
    lib = _lib.load()
    lw = synthetic.make_layer(8900, bits=8)
    h = lw.handle()
    xs = {1: synthetic.make_x(8901, 1, 2048), 40: synthetic.make_x(8902, 40, 2048)}
    bufs = {}
    for T, x in xs.items():
        bufs[T] = (torch.empty_like(x),
                   torch.full((T, 8), -1, dtype=torch.int32, device="cuda"),
                   torch.full((T, 8), -1.0, dtype=torch.float32, device="cuda"),
                   torch.full((1,), 7, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for T, x in xs.items():
            out, idx, sc, st = bufs[T]
            rc = lib.rmoe_moe_block_noalloc(ctypes.byref(h.struct), x.data_ptr(), T, None,
                                            out.data_ptr(), idx.data_ptr(), sc.data_ptr(),
                                            st.data_ptr(), _lib.stream_handle(x.device))
            assert rc == _lib.RMOE_OK, lib.rmoe_last_error()
    torch.cuda.synchronize()
    ref = {}
    for T, x in xs.items():
        ws = torch.zeros(h.workspace_bytes(T), dtype=torch.uint8, device="cuda")
        ref[T] = native.moe_block(h, x, return_routing=True, workspace=ws, check=True)
    for r in range(2):
        for b in bufs.values():
            b[0].zero_()
            b[3].fill_(7)
        g.replay()
        torch.cuda.synchronize()
        for T in xs:
            out, idx, sc, st = bufs[T]
            ro, ri, rs = ref[T]
            assert int(st.item()) == 0, f"replay {r}, {T} tokens: status {int(st.item())}"
            assert torch.equal(idx, ri), f"replay {r}, {T} tokens: indices"
            assert torch.equal(sc, rs), f"replay {r}, {T} tokens: scores"
            assert torch.equal(out, ro), f"replay {r}, {T} tokens: outputs"
        # eager work between the replays
        native.moe_block(h, xs[1], check=True)
        torch.cuda.synchronize()
    print("noalloc capture ok", flush=True)


if __name__ == "__main__":
    main()
