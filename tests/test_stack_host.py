"""Host logic of the persistent decode's launch sequence, on the CPU with
the library call replaced: the token epoch the kernel's counters follow
advances once per launch and not for a launch the library refused."""
import types

import pytest
import torch

from moe_stream_amd import _lib
from moe_stream_amd import geometry as G
from moe_stream_amd.stack import DecodeStack


class _FakeLib:
    def __init__(self):
        self.rc = 0
        self.epochs = []

    def moe_stack_decode(self, *args):
        self.epochs.append(args[18])   # the epoch argument
        return self.rc

    def moe_last_error(self):
        return b"refused before launch"


def _stack_without_device():
    st = object.__new__(DecodeStack)
    st.geom, st.L, st.E, st.k, st.k_pred = G.QWEN3_30B_A3B, 4, 128, 8, 8
    t = torch.zeros(8, dtype=torch.int32)
    st.W = st.table = st.p_ids = st.p_scores = st.p_refs = st.p_pred = st.p_miss = t
    st.p_y = st.p_ws = t
    st.bias = None
    st.pool = types.SimpleNamespace(c_view=lambda: _lib.PoolView())
    st.p_epoch = 0
    return st


def test_refused_launch_does_not_advance_the_epoch(monkeypatch):
    fake = _FakeLib()
    monkeypatch.setattr(_lib, "lib", lambda: fake)
    st = _stack_without_device()
    x = torch.zeros((4, 2048), dtype=torch.bfloat16)
    s = types.SimpleNamespace(cuda_stream=0)
    st.token_persistent(x, stream=s)
    st.token_persistent(x, stream=s)
    fake.rc = _lib.MOE_ERR_INVALID
    with pytest.raises(_lib.MoeError) as ei:
        st.token_persistent(x, stream=s)
    assert ei.value.code == _lib.MOE_ERR_INVALID
    assert st.p_epoch == 2
    fake.rc = 0
    st.token_persistent(x, stream=s)
    assert fake.epochs == [1, 2, 3, 3]
    assert st.p_epoch == 3
