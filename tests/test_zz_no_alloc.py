"""qvex_spec_accept_filtered_bf16_noalloc (static device scratch, no
allocation) against qvex_spec_accept_filtered_bf16 with a caller workspace,
through the C ABI (GPU): two calls in a row, the second smaller, bit-exact
accept counts and tokens; sizes past the scratch are refused on the host."""

import numpy as np
import pytest
import torch

from qvex import _C, kernels
from qvex.kernels import _ptr, _stream

DEV = "cuda:0"


def case(S, k, V, seed):
    g = np.random.default_rng(seed)
    target = (g.standard_normal((S, k + 1, V)) * 3.0).astype(np.float32)
    for s in range(S):
        for i in range(k + 1):
            target[s, i, g.integers(0, V, 3)] += 8.0
    ids = np.argsort(-target[:, :k], axis=-1)[..., 0].astype(np.int32)
    ids[g.random((S, k)) < 0.4] = g.integers(0, V, 1)[0]
    t = torch.from_numpy(target).to(DEV).to(torch.bfloat16)
    return (t, torch.from_numpy(ids).to(DEV), torch.from_numpy(g.random((S, k)).astype(np.float32)).to(DEV),
            torch.from_numpy(g.random(S).astype(np.float32)).to(DEV),
            torch.from_numpy((g.random(V) < 0.05).astype(np.float32)).to(DEV))


def run(noalloc, t, ids, ua, us, seen, S, k, V, top_k, top_p, pen):
    n = torch.full((S,), -7, dtype=torch.int32, device=DEV)
    tok = torch.full((S,), -7, dtype=torch.int32, device=DEV)
    inv = float(np.float32(1.0) / np.float32(0.7))
    args = (_ptr(t), None, _ptr(ids), _ptr(ua), _ptr(us), inv, _ptr(seen), pen, top_k, top_p, _ptr(n), _ptr(tok),
            S, k, V)
    if noalloc:
        _C.call("qvex_spec_accept_filtered_bf16_noalloc", *args, _stream())
    else:
        ws = kernels.spec_workspace(S, k, V, False, DEV, top_k)
        _C.call("qvex_spec_accept_filtered_bf16", *args, _ptr(ws), ws.numel() * 4, _stream())
    torch.cuda.synchronize()
    return n.cpu().numpy(), tok.cpu().numpy()


@pytest.mark.gpu
def test_noalloc_equals_workspace_entry_point():
    # the second call is smaller (fewer steps, drafts and tokens, another filter form)
    for S, k, V, top_k, top_p, pen in ((8, 3, 248320, 20, 0.95, 0.3), (3, 1, 50000, 0, 0.9, 0.0)):
        t, ids, ua, us, seen = case(S, k, V, seed=S * 100 + V % 97)
        a = run(True, t, ids, ua, us, seen, S, k, V, top_k, top_p, pen)
        b = run(False, t, ids, ua, us, seen, S, k, V, top_k, top_p, pen)
        print(f"S={S} k={k} V={V} top_k={top_k}: n {a[0].tolist()} tok {a[1].tolist()}")
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        assert (a[0] >= 0).all() and (a[1] >= 0).all()


@pytest.mark.gpu
def test_noalloc_refuses_sizes_past_the_scratch():
    t = torch.zeros(1, dtype=torch.bfloat16, device=DEV)
    i32 = torch.zeros(1, dtype=torch.int32, device=DEV)
    f = torch.zeros(1, dtype=torch.float32, device=DEV)
    S, k, V, top_k = 64, 7, 248320, 64
    assert _C.lib().qvex_spec_accept_filtered_workspace_bytes(S, k, V, 1, top_k) > (4 << 20)
    with pytest.raises(_C.QvexError, match="static scratch"):
        _C.call("qvex_spec_accept_filtered_bf16_noalloc", _ptr(t), _ptr(t), _ptr(i32), _ptr(f), _ptr(f), 1.0, None,
                0.0, top_k, 0.9, _ptr(i32), _ptr(i32), S, k, V, _stream())
