"""MLA per-head absorbed projections (model.cpp:638-643, 664-665) in one
launch: gpeed_iq3xxs_matvec_heads against the oracle, head by head -- each
head is the reference's own matvec_quant call with row0 = h * rows_per_head on
that head's input vector."""
import numpy as np
import pytest

import gpeed_amd as G
import oracle
from gpeed_amd import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu
TIGHT = 2e-5


def dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


@pytest.mark.parametrize("name,n_heads,rows,in_dim,h0", [
    ("attn_k_b", 64, 512, 256, 0),   # q_abs[h] = W_k[h] q_nope[h]: 64 heads x 512 rows over 256
    ("attn_v_b", 64, 256, 512, 0),   # out[h] = W_v[h] c_comb[h]: 64 heads x 256 rows over 512
    ("attn_k_b_subset", 8, 512, 256, 20),  # heads 20..27 of the tensor (row0 = 20 * 512)
    ("wide", 5, 64, 2048, 1),        # one tile per head, 8 blocks per row
])
def test_matvec_heads(gpu, name, n_heads, rows, in_dim, h0):
    total_heads = h0 + n_heads + 1
    n_rows = total_heads * rows
    w = synth.iq3xxs_matrix(101, n_heads, n_rows, in_dim)
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    x = synth.normal(101, 2, n_heads * in_dim).reshape(n_heads, in_dim)
    x[1] *= np.float32(1e4)  # heads have independent activation scales
    x[2] *= np.float32(1e-5)
    y = G.matvec_heads(t64, n_rows, h0 * rows, in_dim, rows, dev(x, gpu)).cpu().numpy()
    for h in range(n_heads):
        ref = oracle.matvec(w, (h0 + h) * rows, in_dim, rows, x[h])
        assert rel_err(y[h], ref) < TIGHT, (h, rel_err(y[h], ref))


def test_matvec_heads_layout_errors(gpu):
    import torch

    w = synth.iq3xxs_matrix(102, 0, 256, 256)
    t64 = G.tile(dev(w.reshape(-1), gpu), 256, 256)
    x = torch.zeros(2, 256, device=gpu)
    with pytest.raises(G.GpeedError) as e:
        G.matvec_heads(t64, 256, 0, 256, 96, x)
    assert e.value.code == -6
    with pytest.raises(G.GpeedError) as e:
        G.matvec_heads(t64, 256, 64, 256, 128, x)  # rows 64..320 past the tensor
    assert e.value.code == -1
