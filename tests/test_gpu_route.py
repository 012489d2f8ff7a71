"""GPU parity of the one-launch router (T <= 16) where workgroup 0's own
ranking tasks do not see every writer of the launch: 4..16 tokens with the
lookahead router (token 0's lookahead task sits on another workgroup), and a
small expert count with more ranking tasks than router rows (workgroups that
only rank).  Each case runs several launches back to back on one workspace,
so the launch flag (the workspace's sequence word + 1) advances between them;
every launch is checked against the oracle's router and lookahead."""
import numpy as np
import pytest
import torch

from moe_stream_amd import _lib, ops, synth
from moe_stream_amd import geometry as G
from oracle import numerics as N

from helpers import bf16_bits, bf16_randn, bf16_values

pytestmark = pytest.mark.gpu


def _router(E, D, seed):
    g = synth.generator("cuda", seed)
    return (torch.randn((E, D), generator=g, device="cuda") * 0.02).to(torch.bfloat16)


def _check(x, W, Wn, k, kp, table, bufs):
    X = bf16_values(x)
    Z = N.router_logits(X, bf16_bits(W), None, "mlx")
    Zn = N.router_logits(X, bf16_bits(Wn), None, "mlx")
    ids = bufs.ids.cpu().numpy()
    sc = bufs.scores.cpu().numpy().astype(np.float64)
    pred = bufs.pred.cpu().numpy()
    refs = bufs.slot_refs.cpu().numpy()
    for t in range(X.shape[0]):
        rid, rsc, ranked = N.top_k_experts(Z[t], k, True, "mlx")
        assert N.ids_match(ranked, rid, ids[t]), (t, sorted(ids[t]), sorted(rid))
        assert len(set(ids[t].tolist())) == k
        if set(ids[t].tolist()) == set(rid.tolist()):
            by = dict(zip(rid.tolist(), rsc.tolist()))
            exp = np.array([by[int(e)] for e in ids[t]])
            assert np.all(np.abs(sc[t] - exp) <= N.bf16_ulp(exp) * 1.01), (t, sc[t], exp)
        assert N.ids_match(Zn[t], N.top_k_indices(Zn[t], kp), pred[t, :kp]), (t, pred[t])
    np.testing.assert_array_equal(refs, table.cpu().numpy()[ids])


@pytest.mark.parametrize("E,k,kp,T", [(128, 8, 8, 4), (128, 8, 16, 9), (128, 8, 8, 16),
                                      (8, 2, 4, 16), (8, 2, 8, 13), (16, 4, 4, 16)])
def test_route_fused_every_writer_counted(E, k, kp, T):
    D = 2048
    W = _router(E, D, 20260500 + E)
    Wn = _router(E, D, 20260600 + E)
    table = torch.tensor(np.random.default_rng(E).permutation(4 * E)[:E], dtype=torch.int32,
                         device="cuda")
    ws = torch.zeros(_lib.lib().moe_route_workspace(T, E), dtype=torch.uint8, device="cuda")
    bufs = ops.RouteBuffers(T, k, kp, "cuda")
    for rep in range(4):
        x = bf16_randn((T, D), seed=20260700 + 10 * T + rep)
        bufs.pred.fill_(-1)
        bufs.ids.fill_(-1)
        ops.route(x, W, None, _lib.MOE_ROUTE_SOFTMAX_TOPK, True, k, W_next=Wn, k_pred=kp,
                  table=table, bufs=bufs, workspace=ws)
        torch.cuda.synchronize()
        ops.check_device_error()
        _check(x, W, Wn, k, kp, table, bufs)
    # the arrival word is back at zero after every launch
    hdr = ws[:256].view(torch.int32).cpu().numpy()
    assert hdr[32] == 0, hdr[32]
    assert hdr[0] == 4, hdr[0]   # four launches advanced the sequence word
