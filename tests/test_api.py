"""Drop-in API on the CPU: TitanMACConfig, WindowedAttention / MLPBlock /
BlockELLLinear construction and state_dicts, build_band_mask, dense <-> ELL
conversion, meta shapes of the torch ops, and that the hot path refuses CPU
tensors instead of falling back."""
import dataclasses
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn as nn

import titans_core as tc
from oracle import block_ell as ob
from oracle import masks as om
from titans_core.attn.windowed_attention import (WindowConfig, WindowedAttention, build_band_mask,
                                                 convert_mask_to_sdpa_format)
from titans_core.blocks.mlp import MLPBlock
from titans_core.kernels.block_ell import BlockELLLinear, bell_fwd

# Field defaults of the reference dataclass (config.py:80-158).
REFERENCE_DEFAULTS = dict(
    vocab_size=128000, d_model=640, n_heads=10, n_layers=16, d_ff=2560, max_seq_len=4096,
    window_size=512, n_persistent=16, use_block_sparse=True, block_size=64, dropout=0.0,
    tie_weights=True, use_memory_bank=False, enable_test_time_memory=False, memory_mlp_expansion=4,
    memory_lambda_decay=0.95, memory_eta_lr=0.01, memory_rank_ratio=0.25, norm_eps=1e-5,
    attention_dropout=0.0, causal=True, use_neural_memory=False, n_memory_layers=2, d_memory=None,
    memory_theta_lr=0.01, memory_forget_hidden=32, memory_decay_hidden=32, memory_capacity=512,
    titans_variant="MAC", use_parallel_memory=True, segment_size=512, n_memory_tokens=32,
    use_dmgd=False, dmgd_hidden_dim=64, dmgd_n_groups=2, use_cms=False, cms_frequencies=None)


def test_config_defaults_match_reference():
    cfg = tc.TitanMACConfig()
    d = cfg.to_dict()
    for k, v in REFERENCE_DEFAULTS.items():
        assert d[k] == v, k
    new = set(d) - set(REFERENCE_DEFAULTS)
    assert new == {"mlp_block_ell", "mlp_density", "mlp_block_size", "mlp_ell_seed"}
    assert cfg.d_head == 64
    cfg.validate()


@pytest.mark.parametrize("kw,msg", [
    (dict(d_model=641), "must be divisible by n_heads"), (dict(n_persistent=4096), "must be < max_seq_len"),
    (dict(window_size=-1), "window_size must be non-negative"), (dict(d_ff=0), "d_ff must be positive"),
    (dict(dropout=1.5), "dropout must be in"), (dict(memory_lambda_decay=1.0), "memory_lambda_decay"),
    (dict(titans_variant="XYZ"), "titans_variant must be one of"),
    (dict(use_cms=True, cms_frequencies={0: 0}), "CMS frequency must be positive"),
    (dict(mlp_block_ell=True, mlp_density=0.0), "mlp_density"),
    (dict(mlp_block_ell=True, d_ff=2500), "multiple of mlp_block_size")])
def test_config_validate_errors(kw, msg):
    with pytest.raises(ValueError, match=msg):
        tc.TitanMACConfig(**kw).validate()


def test_config_from_cfg_and_repr():
    cfg = tc.TitanMACConfig.from_cfg({"vocab_size": 50000, "d_model": 512, "n_heads": 8, "bogus": 1})
    assert cfg.vocab_size == 50000 and cfg.d_head == 64
    obj = type("O", (), {"d_model": 256, "n_heads": 4})()
    assert tc.TitanMACConfig.from_cfg(obj).d_model == 256
    assert repr(tc.TitanMACConfig()).startswith("TitanMACConfig(d_model=640, n_heads=10")
    with pytest.raises(ValueError):
        tc.TitanMACConfig(d_model=641).d_head


def test_windowed_attention_construction_and_state_dict():
    a = WindowedAttention(WindowConfig(window_size=256, num_heads=8, head_dim=64, n_persistent=16))
    sd = a.state_dict()
    assert set(sd) == {"qkv_proj.weight", "out_proj.weight"}
    assert sd["qkv_proj.weight"].shape == (1536, 512) and sd["out_proj.weight"].shape == (512, 512)
    b = WindowedAttention(tc.TitanMACConfig(d_model=640, n_heads=10, window_size=512))
    assert (b.n_heads, b.d_head, b.window_size, b.num_persistent, b.causal) == (10, 64, 512, 16, True)
    with pytest.raises(AssertionError):
        WindowedAttention(type("C", (), {"d_model": 100, "n_heads": 3, "d_head": 33, "window_size": 4,
                                         "n_persistent": 0, "causal": True, "attention_dropout": 0.0})())


def test_hot_path_refuses_cpu_tensors():
    a = WindowedAttention(WindowConfig(window_size=8, num_heads=2, head_dim=64, n_persistent=2))
    with pytest.raises(RuntimeError, match="runs only on the GPU"):
        a(torch.randn(1, 16, 128))
    with pytest.raises(RuntimeError, match="runs only on the GPU"):
        a(torch.randn(1, 16, 128), attn_mask=torch.ones(16, 16, dtype=torch.bool))
    a.train()
    a.dropout_p = 0.1
    with pytest.raises(RuntimeError, match="runs only on the GPU"):
        a(torch.randn(1, 16, 128))
    lin = BlockELLLinear(128, 128, density=0.5).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="runs only on the GPU"):
        lin(torch.randn(3, 128).to(torch.bfloat16))


@pytest.mark.parametrize("S,w,Np,causal", [(64, 8, 4, True), (100, 30, 0, False), (4096, 512, 16, True),
                                           (17, 100, 16, True)])
def test_build_band_mask_bit_exact(S, w, Np, causal):
    m = build_band_mask(S, w, Np, device="cpu", causal=causal)
    assert m.dtype == torch.bool and m.shape == (S, S)
    assert np.array_equal(m.numpy(), om.band_mask(S, w, Np, causal))
    with pytest.raises(ValueError):
        build_band_mask(8, 2, 8, device="cpu")
    add = convert_mask_to_sdpa_format(m[:8, :8])
    assert add.dtype == torch.float32 and (add[m[:8, :8]] == 0).all() and torch.isinf(add[~m[:8, :8]]).all()


def test_mlp_block_dense_matches_reference_layout():
    m = MLPBlock(128, 512)
    sd = m.state_dict()
    assert {k: tuple(v.shape) for k, v in sd.items()} == {
        "fc1.weight": (512, 128), "fc1.bias": (512,), "fc2.weight": (128, 512), "fc2.bias": (128,)}
    x = torch.randn(2, 3, 128)
    ref = m.fc2(nn.functional.gelu(m.fc1(x)))
    assert torch.allclose(m(x), ref)


def test_mlp_block_ell_construction():
    cfg = tc.TitanMACConfig(d_model=640, d_ff=2560, mlp_block_ell=True, mlp_density=0.5)
    m = MLPBlock.from_config(cfg)
    assert isinstance(m.fc1, BlockELLLinear) and m.fc1.values.shape == (10, 20, 64, 64)
    assert m.fc2.values.shape == (40, 5, 64, 64)
    assert not np.array_equal(m.fc1.col_idx.numpy()[:5, :5], m.fc2.col_idx.numpy()[:5, :5])


def test_block_ell_linear_dense_round_trip_and_pruning():
    torch.manual_seed(0)
    lin = nn.Linear(256, 384)
    e = BlockELLLinear.from_linear(lin, density=0.5, seed=3)
    W = e.to_dense_weight()
    assert W.shape == (384, 256)
    mask = np.kron(ob.block_mask(e.col_idx.numpy(), 6), np.ones((64, 64), dtype=bool)).T  # [out, in]
    assert torch.equal(W[torch.from_numpy(mask)], lin.weight.detach()[torch.from_numpy(mask)])
    assert (W[~torch.from_numpy(mask)] == 0).all()
    back = e.to_linear()
    assert torch.equal(back.weight, W) and torch.equal(back.bias, lin.bias)
    # oracle view of the same layer: values are the [in, out] orientation blocks
    Wkn = ob.to_dense(e.col_idx.numpy(), e.values.detach().numpy(), 6)
    assert np.array_equal(Wkn, W.t().numpy())
    mag = BlockELLLinear.from_linear(lin, width=2, select="magnitude")
    norms = lin.weight.detach().t().reshape(4, 64, 6, 64).pow(2).sum(dim=(1, 3))
    want = np.sort(np.argsort(-norms.numpy(), axis=1, kind="stable")[:, :2], axis=1)
    assert np.array_equal(mag.col_idx.numpy(), want)


def test_block_ell_state_dict_round_trip_with_other_pattern():
    a = BlockELLLinear(128, 256, density=0.5, seed=1)
    b = BlockELLLinear(128, 256, density=0.25, seed=2)
    b.load_state_dict(a.state_dict())
    assert torch.equal(b.col_idx, a.col_idx) and torch.equal(b.values, a.values)
    assert np.array_equal(b.pattern.col_idx, a.col_idx.numpy())


def test_ops_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(2, 7, 128, dtype=torch.bfloat16)
        v = torch.empty(2, 3, 64, 64, dtype=torch.bfloat16)
        i = torch.empty(6, dtype=torch.int32)
        tp = torch.empty(5, dtype=torch.int32)
        y = bell_fwd(x, v, i, tp, i, i, tp[:4], None, False)
        assert y.shape == (2, 7, 256)
        q = torch.empty(2, 3, 100, 64, dtype=torch.bfloat16)
        from titans_core.kernels.window_attn import window_attn_fwd
        o, lse = window_attn_fwd(q, q, q, 8, 2, True, 0, 64, 0.125, True)
        assert o.shape == (2, 100, 3, 64) and lse.shape == (2, 3, 100) and lse.dtype == torch.float32
        from titans_core.kernels.window_attn import window_attn_bwd
        grads = window_attn_bwd(o, q, q, q, o, lse, 8, 2, True, 0, 64, 0.125)
        assert [g.shape for g in grads] == [(2, 3, 100, 64)] * 3


def test_block_sparse_attention_construction_and_state_dict():
    m = tc.BlockSparseAttention(640, 10, window_size=512, block_size=64, n_persistent=16)
    sd = m.state_dict()
    # the reference's keys and shapes (attn/block_sparse_attention.py:84-101)
    assert set(sd) == {"qkv_proj.weight", "conv_q.weight", "conv_k.weight", "conv_v.weight",
                       "out_proj.weight"}
    assert sd["qkv_proj.weight"].shape == (1920, 640) and sd["conv_q.weight"].shape == (640, 1, 4)
    assert set(tc.BlockSparseAttention(128, 2, use_conv=False).state_dict()) == {
        "qkv_proj.weight", "out_proj.weight"}
    with pytest.raises(ValueError, match="divisible"):
        tc.BlockSparseAttention(100, 3)
    cfg = tc.TitanMACConfig()
    m2 = tc.create_block_sparse_attention(cfg)
    assert (m2.block_size, m2.window_size, m2.n_persistent, m2.n_heads) == (64, 512, 16, 10)


def test_block_sparse_attention_refuses_cpu_tensors():
    m = tc.BlockSparseAttention(128, 2, window_size=16, block_size=16, n_persistent=2)
    with pytest.raises(RuntimeError, match="GPU"):
        m(torch.randn(1, 20, 128))


def test_block_ell_linear_loads_dense_checkpoint():
    """A dense nn.Linear state_dict loads into a Block-ELL layer: the pattern stays,
    the stored blocks are the dense weight's blocks at it."""
    torch.manual_seed(1)
    lin = nn.Linear(256, 384)
    e = BlockELLLinear(256, 384, density=0.5, seed=5)
    ci = e.col_idx.clone()
    e.load_state_dict(lin.state_dict())
    assert torch.equal(e.col_idx, ci) and torch.equal(e.bias, lin.bias)
    assert torch.equal(e.values, BlockELLLinear.from_linear(lin, col_idx=ci.numpy()).values)
    with pytest.raises(ValueError, match="does not match"):
        e.load_state_dict(nn.Linear(128, 384).state_dict())


def test_mlp_block_dense_conversions():
    torch.manual_seed(2)
    dense = MLPBlock(128, 256)
    ell = MLPBlock.from_dense(dense, density=0.5, seed=4)
    assert ell.block_ell and ell.fc1.width == 2 and ell.fc2.width == 1
    back = ell.to_dense()
    assert set(back.state_dict()) == set(dense.state_dict())
    assert torch.equal(back.fc1.weight, ell.fc1.to_dense_weight())
    # magnitude pruning of the densified block finds exactly the stored blocks again
    again = MLPBlock.from_dense(back, density=0.5, select="magnitude")
    assert torch.equal(again.fc1.col_idx, ell.fc1.col_idx)
    assert torch.equal(again.fc2.values, ell.fc2.values)
    # and a dense MLP checkpoint loads straight into a Block-ELL MLP (strict)
    cfg = tc.TitanMACConfig(d_model=128, d_ff=256, mlp_block_ell=True, mlp_density=0.5)
    m = MLPBlock.from_config(cfg)
    m.load_state_dict(dense.state_dict())
    assert torch.equal(m.fc1.to_dense_weight(),
                       BlockELLLinear.from_linear(dense.fc1, col_idx=m.fc1.col_idx.numpy())
                       .to_dense_weight())


@pytest.mark.parametrize("block_sparse", [True, False])
def test_titan_block_construction_and_state_dict(block_sparse):
    cfg = tc.TitanMACConfig(d_model=640, n_heads=10, d_ff=2560, use_block_sparse=block_sparse)
    b = tc.TitanBlock(cfg)
    sd = {k: tuple(v.shape) for k, v in b.state_dict().items()}
    # the reference's keys and shapes (blocks/titan_block.py:46-71)
    want = {"norm_attn.scale": (640,), "norm_mlp.scale": (640,),
            "attention.qkv_proj.weight": (1920, 640), "attention.out_proj.weight": (640, 640),
            "mlp.fc1.weight": (2560, 640), "mlp.fc1.bias": (2560,),
            "mlp.fc2.weight": (640, 2560), "mlp.fc2.bias": (640,)}
    if block_sparse:
        want.update({f"attention.conv_{t}.weight": (640, 1, 4) for t in "qkv"})
        assert isinstance(b.attention, tc.BlockSparseAttention)
    else:
        assert isinstance(b.attention, WindowedAttention)
    assert sd == want
    assert b.norm_attn.eps == cfg.norm_eps and torch.equal(b.norm_mlp.scale, torch.ones(640))


def test_titan_block_ell_loads_dense_reference_checkpoint():
    dense = tc.TitanBlock(tc.TitanMACConfig(d_model=128, n_heads=2, d_ff=256))
    ell = tc.TitanBlock(tc.TitanMACConfig(d_model=128, n_heads=2, d_ff=256, mlp_block_ell=True))
    ell.load_state_dict(dense.state_dict())
    assert torch.equal(ell.attention.qkv_proj.weight, dense.attention.qkv_proj.weight)
    assert isinstance(ell.mlp.fc1, BlockELLLinear)


def test_rms_norm_refuses_cpu_tensors():
    with pytest.raises(RuntimeError, match="GPU"):
        tc.RMSNorm(64)(torch.randn(2, 64))


MAC_CFG = dict(vocab_size=61, d_model=64, n_heads=1, n_layers=2, d_ff=128, max_seq_len=128,
               window_size=40, n_persistent=4, block_size=32, use_neural_memory=True,
               segment_size=48, n_memory_tokens=8)


def test_titanmac_state_dict_keys_match_reference_checkpoint():
    """Every key and shape of the reference's TitanMAC state_dict (the golden checkpoint was
    written by the reference module itself) and nothing else."""
    gold = np.load(Path(__file__).parent / "golden" / "mac_golden.npz")
    want = {k[len("state/"):]: gold[k].shape for k in gold.files if k.startswith("state/")}
    m = tc.TitanMAC(tc.TitanMACConfig(**MAC_CFG))
    assert {k: tuple(v.shape) for k, v in m.state_dict().items()} == want
    m.load_state_dict({k: torch.from_numpy(gold[f"state/{k}"]) for k in want})
    assert m.lm_head.weight is m.embed_tokens.weight          # tie_weights
    assert isinstance(m.layers[0].attention, tc.BlockSparseAttention)


def test_titanmac_init_and_param_counts():
    torch.manual_seed(0)
    cfg = tc.TitanMACConfig(**dict(MAC_CFG, tie_weights=False))
    m = tc.TitanMAC(cfg)
    assert abs(float(m.embed_tokens.weight.detach().std()) - 0.02) < 3e-3
    assert m.memory_proj.weight.shape == (64, 64) and m.gate_proj.bias.shape == (64,)
    total = sum(p.numel() for p in m.parameters())
    emb = m.embed_tokens.weight.numel() + m.embed_positions.weight.numel() + m.lm_head.weight.numel()
    assert m.get_num_params(False) == total and m.get_num_params(True) == total - emb
    nm = m.neural_memory
    n = sum(p.numel() for p in nm.memory_mlp.parameters())
    assert nm.momentum_S.shape == (n,) and nm._flat_param_cache.shape == (n,)
    assert [o for o, _ in nm._param_offsets] == [0, 64 * 64, 64 * 64 + 64, 2 * 64 * 64 + 64]
    plain = tc.TitanMAC(tc.TitanMACConfig(**dict(MAC_CFG, use_neural_memory=False)))
    assert plain.neural_memory is None and plain.memory_proj is None
    with pytest.raises(ValueError, match="use_neural_memory"):
        plain.forward_mac(torch.zeros(1, 4, dtype=torch.long))
    with pytest.raises(NotImplementedError):
        tc.TitanMAC(tc.TitanMACConfig(**dict(MAC_CFG, use_memory_bank=True)))


def test_neural_memory_construction_errors_and_cpu_refusal():
    nm = tc.NeuralMemory(d_model=32, n_memory_layers=3, theta_lr=0.1)
    assert len(nm.memory_mlp.linears()) == 3 and nm.theta == 0.1
    for kw, msg in ((dict(d_model=0), "d_model"), (dict(d_model=8, n_memory_layers=0), "n_memory"),
                    (dict(d_model=8, theta_lr=0.0), "theta_lr")):
        with pytest.raises(ValueError, match=msg):
            tc.NeuralMemory(**kw)
    with pytest.raises(ValueError, match="3D"):
        nm.update(torch.zeros(4, 32))
    with pytest.raises(RuntimeError, match="GPU"):
        nm.update(torch.zeros(1, 4, 32))
    # retrieval and the loss are plain torch modules (no HIP op on their path)
    x = torch.randn(2, 5, 32)
    assert nm.retrieve(x).shape == (2, 5, 32) and nm.compute_loss(x).dim() == 0
    from titans_core.kernels import memory_mlp as km
    with pytest.raises(RuntimeError, match="GPU"):
        km.silu_backward(torch.zeros(4), torch.zeros(4))


def test_direct_call_only_when_nothing_is_recorded():
    """The op wrappers skip the torch.library dispatcher only in eager mode, for plain
    tensors, and when no autograd graph has to be recorded for them."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from titans_core.kernels import _lib
    a = torch.zeros(2)
    p = nn.Parameter(torch.zeros(2))
    assert _lib.direct_call(a, None)
    assert not _lib.direct_call(a, p)  # a parameter that needs a gradient
    with torch.no_grad():
        assert _lib.direct_call(a, p)
    with torch.inference_mode():
        assert _lib.direct_call(torch.zeros(2), p)
    p.requires_grad_(False)
    assert _lib.direct_call(a, p)
    with FakeTensorMode() as mode:
        f = mode.from_tensor(a)
    assert not _lib.direct_call(f)


def test_direct_call_defers_to_the_op_under_compile():
    from titans_core.kernels import _lib
    seen = []

    def fn(t):
        seen.append(_lib.direct_call(t))
        return t + 1

    torch.compile(fn, backend="eager")(torch.zeros(2))
    assert seen == [False]
