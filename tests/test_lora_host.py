"""CPU checks of the fused dynamic-LoRA host logic: adapter classification,
concatenation / padding / scale folding, and that the fused pair computes the
sum of the separate adapters' bypass terms."""
import pytest
import torch

from conftest import import_pkg
from fake_comfy import FakeLoHa, FakeLoRA, install_fake_comfy


@pytest.fixture(scope="module")
def ops_mod():
    install_fake_comfy()
    from importlib import import_module, reload
    import_pkg()
    m = import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = reload(m)
    return m


def _adapter(N, K, r, alpha, seed, cls=FakeLoRA, mult=1.0):
    g = torch.Generator().manual_seed(seed)
    v = cls(torch.randn(N, r, generator=g) * 0.05, torch.randn(r, K, generator=g) * 0.05, alpha)
    v.multiplier = mult
    return v


def test_fuse_pairs_layout_and_padding(backend):
    N, K = 40, 96
    a = _adapter(N, K, 8, 4.0, 1)
    b = _adapter(N, K, 16, None, 2)
    pa = (a.weights[1], a.weights[0], 0.75 * 4.0 / 8)
    pb = (b.weights[1], b.weights[0], 1.0)
    D, U = backend.fuse_lora_pairs([pa, pb])
    assert D.shape == (32, K) and U.shape == (N, 32)
    assert D.dtype == torch.bfloat16 and U.dtype == torch.bfloat16
    torch.testing.assert_close(D[:8].float(), pa[0].to(torch.bfloat16).float(), rtol=0, atol=0)
    torch.testing.assert_close(D[8:24].float(), pb[0].to(torch.bfloat16).float(), rtol=0, atol=0)
    assert torch.count_nonzero(D[24:]) == 0 and torch.count_nonzero(U[:, 24:]) == 0
    torch.testing.assert_close(U[:, :8].float(), (pa[1] * pa[2]).to(torch.bfloat16).float(), rtol=0, atol=0)


def test_fused_product_is_sum_of_adapter_terms(backend):
    """(x D^T) U^T over the concatenation equals the sum of each adapter's
    scaled up(down(x)) (up to the bf16 storage of D and U)."""
    N, K = 64, 128
    ads = [_adapter(N, K, 16, 8.0, 3, mult=0.5), _adapter(N, K, 32, 16.0, 4, mult=1.25),
           _adapter(N, K, 4, None, 5)]
    x = torch.randn(7, K, generator=torch.Generator().manual_seed(6))
    want = sum(v.h(x, torch.empty(0)) for v in ads)
    pairs = [(v.weights[1], v.weights[0], v.multiplier * (v.weights[2] / 16 if i == 0 else
                                                          v.weights[2] / 32 if i == 1 else 1.0))
             for i, v in enumerate(ads)]
    D, U = backend.fuse_lora_pairs(pairs)
    assert D.shape[0] == 64
    got = (x @ D.float().T) @ U.float().T
    err = (got - want).norm() / want.norm()
    assert err < 1e-2, err


def test_fuse_pairs_rank_limit_and_errors(backend):
    N, K = 16, 64
    big = [(torch.zeros(100, K), torch.zeros(N, 100), 1.0), (torch.zeros(29, K), torch.zeros(N, 29), 1.0)]
    assert backend.fuse_lora_pairs(big) is None                      # 129 -> 160 > 128
    assert backend.fuse_lora_pairs([]) is None
    with pytest.raises(ValueError):
        backend.fuse_lora_pairs([(torch.zeros(8, K), torch.zeros(N, 8), 1.0),
                                 (torch.zeros(8, K + 16), torch.zeros(N, 8), 1.0)])


def test_plain_lora_classification(ops_mod):
    N, K = 48, 512
    v = _adapter(N, K, 8, 16.0, 7, mult=0.5)
    down, up, s = ops_mod._plain_lora(v, K, N)
    assert down is v.weights[1] and up is v.weights[0] and s == pytest.approx(0.5 * 16.0 / 8)
    assert ops_mod._plain_lora(_adapter(N, K, 8, None, 7), K, N)[2] == 1.0
    assert ops_mod._plain_lora(_adapter(N, K, 8, 1.0, 7, cls=FakeLoHa), K, N) is None
    assert ops_mod._plain_lora(v, K + 16, N) is None                  # does not fit the layer
    mid = FakeLoRA(v.weights[0], v.weights[1], 1.0, mid=torch.zeros(8, 8))
    assert ops_mod._plain_lora(mid, K, N) is None
    dora = FakeLoRA(v.weights[0], v.weights[1], 1.0, dora_scale=torch.ones(N))
    assert ops_mod._plain_lora(dora, K, N) is None


def test_set_dyn_lora_splits_plain_and_other(ops_mod):
    N, K = 48, 512
    lin = ops_mod.Int4ConvRotOps.Linear(K, N, bias=False)
    plain = _adapter(N, K, 8, 8.0, 8)
    other = _adapter(N, K, 8, 8.0, 9, cls=FakeLoHa)
    lin._set_dyn_lora([plain, other])
    assert lin._dyn_lora == [plain, other]
    D, U = lin._dyn_fused
    assert D.shape == (32, K) and U.shape == (N, 32)
    assert lin._dyn_rest == [other]
    lin._set_dyn_lora([other])
    assert lin._dyn_fused is None and lin._dyn_rest == [other]
