"""2-bit E8 compression of optimizer state (ojasx2/grad_free_optimizer.py:106-157): the
state keys, padding and round trip of the reference's helpers, with packed bytes and
decoded values bit-exact with the CPU oracle."""

import numpy as np
import pytest
import torch

from ojasx_amd import optim_state as S
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("shape", [(37, 19), (64, 32), (9,), (8,)])
def test_exp_avg_pack_round_trip_matches_oracle(shape):
    g = torch.Generator().manual_seed(sum(shape))
    m = torch.randn(*shape, generator=g) * 1e-3
    st = {"step": 3, "exp_avg": torch.zeros(shape)}
    S.pack_exp_avg(st, m.to(DEV), use_e8=True, storage_dtype=torch.float32)
    assert "exp_avg" not in st and st["exp_avg_packed"].device.type == "cuda"
    n = m.numel()
    rows = (n + 31) // 32
    assert st["exp_avg_padded_rows"] == rows
    flat = np.zeros(rows * 32, dtype=np.float32)
    flat[:n] = m.reshape(-1).numpy()
    pk, sc, _ = O.e8b_encode(flat, 32)
    assert np.array_equal(st["exp_avg_packed"].cpu().numpy(), pk)
    assert np.array_equal(st["exp_avg_scales"].cpu().view(torch.int16).numpy().view(np.uint16), sc)
    out = S.unpack_exp_avg(st, torch.Size(shape), torch.float32)
    assert out.shape == shape
    ref = O.e8b_decode(pk, sc, rows * 32, 32, O.DT_F32)[:n].reshape(shape)
    assert np.array_equal(out.cpu().numpy(), ref)


def test_small_or_dense_exp_avg_stays_dense():
    st = {}
    t = torch.randn(5, device=DEV)
    S.pack_exp_avg(st, t, use_e8=True, storage_dtype=torch.bfloat16)  # fewer than 8 values
    assert st["exp_avg"].dtype == torch.bfloat16 and "exp_avg_packed" not in st
    keep = st["exp_avg"]
    S.pack_exp_avg(st, t * 2, use_e8=False, storage_dtype=torch.bfloat16)
    assert st["exp_avg"] is keep  # overwritten in place
    assert torch.equal(S.unpack_exp_avg(st, torch.Size([5]), torch.float32),
                       (t * 2).to(torch.bfloat16).float())


def test_grad_accum_is_always_packed():
    st = {"grad_accum": torch.ones(10)}
    g = torch.randn(4, 10, device=DEV)
    S.pack_grad_accum(st, g)
    assert "grad_accum" not in st and st["grad_accum_padded_rows"] == 2
    out = S.unpack_grad_accum(st, g.shape, torch.float32)
    assert out.shape == g.shape
    assert torch.nn.functional.cosine_similarity(out.reshape(-1), g.reshape(-1), dim=0) > 0.9
