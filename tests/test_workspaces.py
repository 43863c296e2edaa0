"""Host-side workspace cache of the op (grinqh/kernel.py ``_Workspaces``):
power-of-two growth, outgrown buffers dropped unless a graph captured them,
and the retired bytes bounded by the live size.  CPU tensors stand in for
device memory; the capture state is injected."""
import torch

from grinqh.kernel import _Workspaces

CPU = torch.device("cpu")


def test_rising_sizes_keep_no_retired_buffer():
    ws = _Workspaces(capturing=lambda dev: False)
    last = None
    for n in range(1, 200):
        buf = ws.get(CPU, 0, n * 37_000)
        assert buf.numel() >= n * 37_000
        assert buf.numel() & (buf.numel() - 1) == 0  # a power of two
        last = buf
    assert ws.retired_bytes() == 0
    assert last.numel() <= 2 * 199 * 37_000


def test_same_size_class_reuses_the_buffer():
    ws = _Workspaces(capturing=lambda dev: False)
    a = ws.get(CPU, 0, 3 << 20)
    b = ws.get(CPU, 0, 4 << 20)
    assert a.data_ptr() == b.data_ptr()
    assert ws.get(CPU, 0, 0) is None
    assert ws.get(CPU, 1, 1).data_ptr() != a.data_ptr()  # another stream, another buffer


def test_only_captured_buffers_are_retired_and_bounded():
    state = {"capturing": False}
    ws = _Workspaces(capturing=lambda dev: state["capturing"])
    sizes = [1 << 20, 3 << 20, 9 << 20, 17 << 20, 40 << 20]
    for i, n in enumerate(sizes):
        buf = ws.get(CPU, 0, n)  # eager call: grows
        state["capturing"] = True
        assert ws.get(CPU, 0, n).data_ptr() == buf.data_ptr()  # captured while current
        state["capturing"] = False
        live = buf.numel()
        assert ws.retired_bytes() < live
    assert ws.retired_bytes() == sum(ws._size_for(n) for n in sizes[:-1])


def test_growth_during_capture_is_refused():
    state = {"capturing": False}
    ws = _Workspaces(capturing=lambda dev: state["capturing"])
    ws.get(CPU, 0, 1 << 20)
    state["capturing"] = True
    try:
        ws.get(CPU, 0, 8 << 20)
    except RuntimeError as e:
        assert "before graph capture" in str(e)
    else:
        raise AssertionError("growing the workspace under capture must raise")
