"""The single-launch decode's hand-overs under conditions that used to break
them, run on the GPU through the C ABI (native wrappers):

* plain launches queued right behind kernels of a few workgroups, after
  which the dispatcher starts the launch on another XCD than 0 (the kernel
  takes each workgroup's XCD from the hardware);
* a call cancelled from the host through the abort word: every workgroup
  skips its waits, the call returns promptly, the status word reads 1, and
  the next call on the workspace is correct;
* the 16-bit phase tags wrapping around, and a call with more routed slots
  after calls with fewer (every hand-over word is rewritten in every layer,
  so no word left by an older call can carry the current tag);
* the few-token router's tagged logits across the wrap, and cancelled.

Outputs are compared bit for bit with the same calls made in the ordinary
way (cooperative launches, fresh epochs), which the oracle tests pin."""

import ctypes
import time

import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runnel_amd import _lib
    _lib.load()
    return torch


@pytest.fixture(scope="module")
def layer8(torch_cuda):
    from runnel_amd import synthetic
    lw = synthetic.make_layer(6100, bits=8)
    return lw, lw.handle()


def _words(ws, torch):
    """(epoch, status, abort) words of a workspace's single-launch scratch
    (rmoe.h: the epoch precedes the status word, the abort word follows)."""
    from runnel_amd import _lib
    off = _lib.load().rmoe_workspace_status_offset()
    return ws[off - 4:off + 8].view(torch.int32)


def test_plain_launches_behind_small_kernels(torch_cuda, layer8):
    """Plain launches (as a captured graph makes them) queued without a sync
    right behind 3- and 7-workgroup kernels give the cooperative outputs bit
    for bit and leave the status word clear."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    _, h = layer8
    xs = synthetic.make_x(6101, 8, 2048)
    ws = torch.zeros(h.workspace_bytes(1), dtype=torch.uint8, device="cuda")
    prev = native.set_cooperative_launch(True)
    try:
        ref = [native.moe_block(h, xs[t:t + 1], workspace=ws, check=False) for t in range(8)]
        torch.cuda.synchronize()
    finally:
        native.set_cooperative_launch(prev)
    assert native.workspace_status(ws) == 0
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    part = torch.zeros(8, dtype=torch.int32, device="cuda")
    got = []
    prev = native.set_cooperative_launch(False)
    try:
        for t in range(8):
            native.stream_read(buf, 3 if t % 2 else 7, part)
            got.append(native.moe_block(h, xs[t:t + 1], workspace=ws, check=False))
        torch.cuda.synchronize()
    finally:
        native.set_cooperative_launch(prev)
    print(f"plain launches behind small kernels: status {native.workspace_status(ws)}",
          flush=True)
    assert native.workspace_status(ws) == 0
    for t in range(8):
        assert torch.equal(got[t], ref[t]), f"token {t}"


def test_cancelled_call_ends_promptly(torch_cuda, layer8):
    """The host writes the next call's key (epoch + 1) into the abort word:
    a 24-layer chained call then waits for nothing, ends in about the time
    of an ordinary call, and sets the status word to 1; after clearing it,
    the next call matches an uncancelled one."""
    torch = torch_cuda
    from runnel_amd import _lib, native, synthetic
    _, h = layer8
    chain = native.Chain([h] * 24)
    ws = torch.zeros(chain.workspace_bytes(), dtype=torch.uint8, device="cuda")
    x = synthetic.make_x(6102, 1, 2048)
    ref = native.moe_chain(chain, x, workspace=ws, check=False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    native.moe_chain(chain, x, workspace=ws, check=False)
    torch.cuda.synchronize()
    t_ok = time.perf_counter() - t0
    w = _words(ws, torch)
    epoch = int(w[0].item())
    assert int(w[1].item()) == 0
    w[2].fill_(epoch + 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    native.moe_chain(chain, x, workspace=ws, check=False)
    torch.cuda.synchronize()
    t_cancel = time.perf_counter() - t0
    print(f"cancelled call {t_cancel * 1e6:.0f} us, ordinary call {t_ok * 1e6:.0f} us",
          flush=True)
    assert native.workspace_status(ws) == 1
    assert t_cancel < max(20 * t_ok, 0.05)
    with pytest.raises(_lib.RmoeError) as e:
        native.check_status(ws)
    assert e.value.status == _lib.RMOE_ETIMEOUT
    again = native.moe_chain(chain, x, workspace=ws, check=False)
    torch.cuda.synchronize()
    assert native.workspace_status(ws) == 0
    assert torch.equal(again, ref)


def test_tag_wrap_and_more_slots_after_fewer(torch_cuda, layer8):
    """Calls across the 65535-phase wrap of the tags equal the same calls at
    a fresh epoch; a top-8 call whose tags equal those of an older top-8
    call, made after top-4 calls on the same workspace, equals the first."""
    torch = torch_cuda
    from runnel_amd import _lib, native, synthetic
    _, h = layer8
    s4 = _lib.Layer.from_buffer_copy(h.struct)
    s4.top_k = 4
    h4 = native.LayerHandle(s4, h.tensors)
    x = synthetic.make_x(6103, 1, 2048)
    ws = torch.zeros(h.workspace_bytes(1), dtype=torch.uint8, device="cuda")
    w = _words(ws, torch)
    # epoch 0: phase 1
    a8 = native.moe_block(h, x, workspace=ws, check=False).clone()
    a4 = native.moe_block(h4, x, workspace=ws, check=False).clone()
    torch.cuda.synchronize()
    # the next call's phase 65536 has the tag of phase 1
    w[0].fill_(65535)
    b8 = native.moe_block(h, x, workspace=ws, check=False)
    b4 = native.moe_block(h4, x, workspace=ws, check=False)
    torch.cuda.synchronize()
    assert native.workspace_status(ws) == 0
    assert torch.equal(b8, a8)
    assert torch.equal(b4, a4)
    # a 12-layer chain whose phases cross 65535 -> 1
    chain = native.Chain([h] * 12)
    ws2 = torch.zeros(chain.workspace_bytes(), dtype=torch.uint8, device="cuda")
    ref = native.moe_chain(chain, x, workspace=ws2, check=False).clone()
    torch.cuda.synchronize()
    _words(ws2, torch)[0].fill_(65529)
    got = native.moe_chain(chain, x, workspace=ws2, check=False)
    torch.cuda.synchronize()
    assert native.workspace_status(ws2) == 0
    assert torch.equal(got, ref)


def test_deferred_status_check_raises_within_the_period(torch_cuda, layer8):
    """Eager one-token calls check the status word without waiting: a set
    word is reported by a later eager call, within one period of the copies
    (every 32nd call) after it was set, and the word is cleared."""
    torch = torch_cuda
    from runnel_amd import _lib, native, synthetic
    _, h = layer8
    ws = torch.zeros(h.workspace_bytes(1), dtype=torch.uint8, device="cuda")
    x = synthetic.make_x(6104, 1, 2048)
    native.moe_block(h, x, workspace=ws)
    torch.cuda.synchronize()
    _words(ws, torch)[1].fill_(1)       # as a failed call leaves it
    torch.cuda.synchronize()
    raised_at = None
    for i in range(2 * native._STATUS.every + 2):
        try:
            native.moe_block(h, x, workspace=ws)
            torch.cuda.synchronize()
        except _lib.RmoeError as e:
            assert e.status == _lib.RMOE_ETIMEOUT
            raised_at = i
            break
    print(f"deferred check raised at call {raised_at}", flush=True)
    assert raised_at is not None and raised_at <= native._STATUS.every + 1
    assert native.workspace_status(ws) == 0
    native.moe_block(h, x, workspace=ws)
    torch.cuda.synchronize()
    assert native.workspace_status(ws) == 0


def test_few_token_router_hand_over(torch_cuda):
    """The few-token router hands its logits over as tagged words: 4-token
    calls across the 65535-phase wrap of the tags equal the first call bit
    for bit; a call cancelled through the abort word returns promptly with
    the status word at 1, and the next call is correct again."""
    torch = torch_cuda
    from runnel_amd import _lib, native, synthetic
    lw = synthetic.make_layer(6200, bits=8)
    h = lw.handle()
    x = synthetic.make_x(6201, 4, 2048)
    ws = torch.zeros(h.workspace_bytes(4), dtype=torch.uint8, device="cuda")
    ref = native.moe_block(h, x, workspace=ws, check=False).clone()
    torch.cuda.synchronize()
    assert native.workspace_status(ws) == 0
    w = _words(ws, torch)
    w[0].fill_(65532)
    for i in range(5):
        got = native.moe_block(h, x, workspace=ws, check=False)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"call {i} across the wrap"
    assert native.workspace_status(ws) == 0
    t0 = time.perf_counter()
    native.moe_block(h, x, workspace=ws, check=False)
    torch.cuda.synchronize()
    t_ok = time.perf_counter() - t0
    epoch = int(w[0].item())
    w[2].fill_(epoch + 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    native.moe_block(h, x, workspace=ws, check=False)
    torch.cuda.synchronize()
    t_cancel = time.perf_counter() - t0
    print(f"cancelled 4-token call {t_cancel * 1e6:.0f} us, ordinary {t_ok * 1e6:.0f} us",
          flush=True)
    assert t_cancel < max(20 * t_ok, 0.05)
    with pytest.raises(_lib.RmoeError) as e:
        native.check_status(ws)
    assert e.value.status == _lib.RMOE_ETIMEOUT
    again = native.moe_block(h, x, workspace=ws, check=False)
    torch.cuda.synchronize()
    assert native.workspace_status(ws) == 0
    assert torch.equal(again, ref)


def test_few_token_words_apart_from_other_routers(torch_cuda):
    """The few-token router's tagged words have an area of their own: a
    general-path call on the same workspace leaves its fp32 logits and int32
    expert ids (small integers, which equal a tag at the right epoch) where
    it keeps them, and a few-token call whose tag equals each such id still
    equals the same call on a fresh workspace."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    from helpers import dev_bf16, layer_to_dev
    from oracle import moe_ref as M
    few = synthetic.make_layer(6300, bits=8)
    hf = few.handle()
    small = layer_to_dev(M.make_layer(6301, hidden=512, inter=128, experts=32, top_k=4, bits=8))
    xf = synthetic.make_x(6302, 4, 2048)
    xs = dev_bf16(M.make_x(6303, 4, 512))
    need = max(hf.workspace_bytes(4), small.workspace_bytes(4))
    ref = native.moe_block(hf, xf, workspace=torch.zeros(need, dtype=torch.uint8, device="cuda"),
                           check=False).clone()
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    w = _words(ws, torch)
    _, idx, _ = native.moe_block(small, xs, workspace=ws, return_routing=True, check=False)
    torch.cuda.synchronize()
    ids = sorted({int(v) for v in idx.flatten().tolist() if int(v) >= 2})
    assert ids
    for e in ids[:6]:
        native.moe_block(small, xs, workspace=ws, check=False)
        torch.cuda.synchronize()
        w[0].fill_(e - 2)  # the next few-token call's tag is e
        got = native.moe_block(hf, xf, workspace=ws, check=False)
        torch.cuda.synchronize()
        assert native.workspace_status(ws) == 0
        assert torch.equal(got, ref), f"tag {e}"
