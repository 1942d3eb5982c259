"""Benchmark of the TitanMAC sparse hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--mode MODE]

A step is one pass of the hot path over one batch of synthetic input. The
headline `value` is the Block-ELL SpMM forward of BASELINE config 2 (X [8192,
2560] bf16 · W [2560, 10240] Block-ELL, 64x64 blocks, 40 of 160 block-columns
per block-row), in effective TFLOP/s (multiply-adds on stored blocks only).
The same run also times, as secondary figures:
  - the dense bf16 GEMM of the same layer (the reference's nn.Linear, hipBLASLt), for the
    speed-up of the Block-ELL forward over it;
  - windowed attention forward of config 3 (B=8, H=10, S=4096, dh=64, w=512,
    Np=16, bf16) in tokens/s, against the dense masked SDPA and the dense
    bmm -> softmax -> bmm path on the same GPU (the faster one is the
    denominator of `attn_speedup_vs_dense`); also at the model-shaped S=4112
    (4096 tokens + 16 persistent) and with BlockSparseAttention's block-window
    mask (block 64);
  - config 1 on the GPU: the fp32 WindowedAttention module (B=2, T=512, d=512, 8 heads,
    w=256, Np=16; qkv GEMM -> fp32 tile kernel -> out GEMM), beside its CPU timing, and
    its forward + backward;
  - the windowed attention backward (dQ, dK, dV) of config 3, against a dense
    masked bf16 backward (five bmm over the full S x S);
  - Block-ELL dX and dW-SDDMM of config 4 (M=32768, W [640, 2560], width 20 of 40), and one
    bf16 training step (forward + backward) of a Block-ELL MLPBlock 640 -> 2560 -> 640 at
    that shape;
  - the causal depthwise conv of BlockSparseAttention (B=8, T=4096, 1920 channels,
    4 taps) and TitanBlock's RMSNorm (32768 x 640), forward and backward, in GB/s
    of compulsory HBM traffic;
  - config 5: the full TitanMAC forward (MAC variant, 16 layers, d_model 640, 10 heads,
    window 512, 16 persistent tokens, 32 memory tokens per 512-token segment, Block-ELL
    MLP at 50%, vocab 50000, random init) on token ids [4, 4096] in bf16, eval, in
    tokens/s; once with the read-only memory of the default config (segments batched),
    once with test-time memory on (segments in order, one memory update each), and once
    more so with each segment's layer stack replayed from a captured HIP graph;
  - the neural-memory update step (norm, clip, momentum, forgetting) over config 5's
    memory MLP (2 x 640 x 640 + biases, fp32) in GB/s of compulsory traffic.
Inputs are drawn on the CPU from fixed seeds and copied to HBM before timing.
Kernel time is measured with HIP events on the launch stream (torch's current
stream) around exactly K back-to-back launches after W warm-up launches, with a
device synchronisation on both sides; ms_per_step is that time over K.
The CPU baseline runs the oracle's dense restatement of the reference path
(X @ to_dense(W) in fp32 numpy) on the host cores, rank 0 only; the reference-equivalent
PyTorch paths of configs 1, 3 and 4 are timed on the CPU as secondary figures.
roofline.traffic is measured by the run itself: two rocprofv3 counter passes (FETCH_SIZE,
WRITE_SIZE) over `--mode traffic` of the current build, scaled by a plain 1 GiB copy.

Modes (for profiling runs): all (default), spmm, attn, attn_cfg1, attn_bwd, attn_ex, dx, sddmm, bell_f32,
mlp_train, conv, norm, mac, mac_ttm, memupd, copy (a plain 1 GiB device copy, used to scale rocprofv3's FETCH_SIZE / WRITE_SIZE),
traffic (the copy then the SpMM, three launches each: what the counter passes profile).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "titanmac-standalone_amd"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from titans_core.kernels import _lib  # noqa: E402
from titans_core.kernels.block_ell import BlockELLPattern, _sddmm_workspace_bytes  # noqa: E402
from titans_core.kernels.window_attn import (_device_work_list, _device_work_list_kv,  # noqa: E402
                                             window_attn_fwd)

METRIC = "Block-ELL SpMM effective TFLOP/s; windowed-attn fwd tokens/s at T=4096,w=512"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
BS = 64

CFG2 = dict(M=8192, n_brow=40, n_bcol=160, width=40, seed=0)
TRAFFIC_REPS = 3  # launches of the copy and of the SpMM in --mode traffic
CFG3 = dict(B=8, H=10, S=4096, dh=64, window=512, n_persistent=16, seed=3)
CFG4 = dict(M=32768, n_brow=10, n_bcol=40, width=20, seed=4)


def band_pairs(S: int, w: int, Np: int) -> int:
    """Allowed (query, key) pairs of the causal band mask with Np persistent tokens."""
    T = S - Np
    a = min(T, w + 1)
    return Np * Np + T * Np + a * (a - 1) // 2 + (T - a) * w + T


CLOCK_SETTLE_S = 0.1  # untimed load before the headline's warmup (see settle)


def settle(launch, seconds: float) -> None:
    """Back-to-back launches of the workload for `seconds` of wall time, untimed. An
    MI355X coming out of idle runs its first ≈ 10–20 ms of load below its sustained
    clock (the SpMM's first block of launches after even a 2 s pause takes ≈ 160 µs
    per launch, the following ones 133–144 µs), so without this the timed steps would
    measure the ramp from idle rather than the throughput of a running job."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            launch()
        torch.cuda.synchronize()


def timed(launch, steps: int, warmup: int, stream) -> float:
    """Mean ms per launch over exactly `steps` back-to-back launches after `warmup`
    untimed ones: the device is synchronised, one HIP event is recorded on the launch
    stream (torch's current stream, where the kernels go) before the first timed launch
    and one after the last, and the device is synchronised again. Nothing is inserted
    between the launches, so this is the whole job's rate."""
    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps):
        launch()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def gen(shape, seed, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


# ---------------------------------------------------------------------------
# Workloads (each returns a zero-argument launch closure and its work figures)
# ---------------------------------------------------------------------------

def setup_spmm(dev):
    from titans_core.kernels import block_ell as kbe
    c = CFG2
    pat = BlockELLPattern.sample(c["seed"], c["n_brow"], c["n_bcol"], c["width"])
    K, N = BS * c["n_brow"], BS * c["n_bcol"]
    X_cpu = gen((c["M"], K), c["seed"] + 1)
    V_cpu = gen((c["n_brow"], c["width"], BS, BS), c["seed"] + 2, 0.02)
    X, V = X_cpu.to(dev), V_cpu.to(dev)
    Y = torch.empty(c["M"], N, dtype=torch.bfloat16, device=dev)
    idx = pat.device_index(dev)
    L = _lib.lib()
    stream = _lib.stream_ptr(dev)
    args = (_lib.ptr(X), K, _lib.ptr(V), _lib.ptr(idx["t_ptr"]), _lib.ptr(idx["t_row"]),
            _lib.ptr(idx["t_vblk"]), _lib.ptr(idx["order"]), _lib.ptr(None), _lib.ptr(Y), N,
            c["M"], c["n_brow"], c["n_bcol"], c["width"], _lib.BF16, _lib.EPI_NONE, stream)
    # the headline path: the grouped forward (block-column pairs sharing block-rows, one
    # activation-tile copy per union step), what block_ell_mm runs at this shape
    # (tiles spread over the persistent workgroups in the pattern's balanced order)
    tord = pat.tile_order(c["M"], dev)
    ga = kbe._grouped_args(idx["grp"], c["M"], K, c["n_bcol"], torch.bfloat16, tord)
    assert ga is not None, "config 2 is expected to take the grouped forward"
    gargs = (_lib.ptr(X), K, _lib.ptr(V), ga[0], ga[1], ga[2], ga[3], 2, ga[4], ga[5], _lib.ptr(None),
             _lib.ptr(Y), N, c["M"], c["n_brow"], c["n_bcol"], c["width"], _lib.BF16, _lib.EPI_NONE, stream)

    def launch():
        rc = L.tmac_bell_fwd_grouped(*gargs)
        if rc:
            _lib.check(rc, "tmac_bell_fwd_grouped")

    # the same grouped kernel with its tiles dealt round-robin (secondary figure)
    gargs_rr = gargs[:8] + (None, 0) + gargs[10:]

    def launch_rr():
        rc = L.tmac_bell_fwd_grouped(*gargs_rr)
        if rc:
            _lib.check(rc, "tmac_bell_fwd_grouped")

    # the per-block-column gather kernel on the same layer (secondary figure)
    def launch_gather():
        rc = L.tmac_bell_fwd(*args)
        if rc:
            _lib.check(rc, "tmac_bell_fwd")

    # the same layer on its first 64 rows only (a decoding-sized batch: the few-row kernel)
    args_m64 = args[:10] + (64,) + args[11:]

    def launch_m64():
        rc = L.tmac_bell_fwd(*args_m64)
        if rc:
            _lib.check(rc, "tmac_bell_fwd")

    nnz = c["n_brow"] * c["width"]
    flops = 2 * c["M"] * nnz * BS * BS
    bytes_ = c["M"] * K * 2 + nnz * BS * BS * 2 + (c["n_bcol"] + 1 + 2 * nnz + c["n_bcol"]) * 4 + c["M"] * N * 2
    return dict(launch=launch, launch_rr=launch_rr, launch_gather=launch_gather, launch_m64=launch_m64,
                weight_bytes=nnz * BS * BS * 2, flops=flops,
                bytes=bytes_, pat=pat, X_cpu=X_cpu, V_cpu=V_cpu, keep=(X, V, Y, idx))


def setup_bell_f32(dev):
    """The fp32 Block-ELL path (fp32 MFMA): forward at config 2's shape, dX and SDDMM at
    config 4's, fp32 inputs and outputs."""
    from titans_core.kernels import block_ell as kbe
    out = {}
    c = CFG2
    pat = BlockELLPattern.sample(c["seed"], c["n_brow"], c["n_bcol"], c["width"])
    X = gen((c["M"], BS * c["n_brow"]), c["seed"] + 1, dtype=torch.float32).to(dev)
    V = gen((c["n_brow"], c["width"], BS, BS), c["seed"] + 2, 0.02, dtype=torch.float32).to(dev)
    idx = pat.device_index(dev)
    out["fwd"] = lambda: kbe._bell_fwd(X, V, idx["col_idx"], idx["t_ptr"], idx["t_row"],
                                       idx["t_vblk"], idx["order"], None, False)
    out["fwd_flops"] = 2 * c["M"] * c["n_brow"] * c["width"] * BS * BS
    c4 = CFG4
    pat4 = BlockELLPattern.sample(c4["seed"], c4["n_brow"], c4["n_bcol"], c4["width"])
    X4 = gen((c4["M"], BS * c4["n_brow"]), c4["seed"] + 1, dtype=torch.float32).to(dev)
    dY4 = gen((c4["M"], BS * c4["n_bcol"]), c4["seed"] + 2, dtype=torch.float32).to(dev)
    V4 = gen((c4["n_brow"], c4["width"], BS, BS), c4["seed"] + 3, 0.02, dtype=torch.float32).to(dev)
    idx4 = pat4.device_index(dev)
    out["dx"] = lambda: kbe._bell_dx(dY4, V4, idx4["col_idx"], c4["n_bcol"])
    out["sddmm"] = lambda: kbe._bell_sddmm(X4, dY4, idx4["col_idx"], c4["n_brow"], c4["width"],
                                           torch.float32)
    out["bwd_flops"] = 2 * c4["M"] * c4["n_brow"] * c4["width"] * BS * BS
    out["keep"] = (X, V, idx, X4, dY4, V4, idx4)
    return out


def setup_mlp_train(dev):
    """One training step (forward + backward) of a bf16 Block-ELL MLPBlock at config 4's
    shape: 640 -> 2560 -> 640 at 50% density, 32768 rows; fc1 + GELU through the fused
    training path (tmac_bell_fwd_gelu_aux, tmac_bell_gelu_bwd)."""
    from titans_core.blocks.mlp import MLPBlock
    c4 = CFG4
    torch.manual_seed(c4["seed"])
    m = MLPBlock(BS * c4["n_brow"], BS * c4["n_bcol"], block_ell=True, density=0.5,
                 seed=c4["seed"]).to(dev, torch.bfloat16).train()
    x = gen((c4["M"], BS * c4["n_brow"]), c4["seed"] + 1).to(dev).requires_grad_(True)
    gy = gen((c4["M"], BS * c4["n_brow"]), c4["seed"] + 2).to(dev)

    def launch():
        x.grad = None
        m.zero_grad(set_to_none=True)
        m(x).backward(gy)
    nnz = m.fc1.pattern.nnz_blocks + m.fc2.pattern.nnz_blocks
    return dict(launch=launch, flops=3 * 2 * c4["M"] * nnz * BS * BS, keep=(m, x, gy))


def setup_attn(dev, S=None, pattern=None, block_size=64):
    """Windowed attention forward at config 3's shape (S overridable; the pattern
    defaults to the band of WindowedAttention)."""
    c = dict(CFG3)
    if S is not None:
        c["S"] = S
    pattern = _lib.PATTERN_BAND if pattern is None else pattern
    shape = (c["B"], c["S"], 3, c["H"], c["dh"])  # fused qkv projection output layout
    qkv = gen(shape, c["seed"]).to(dev)
    q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))  # [B, H, S, dh] views
    out = torch.empty(c["B"], c["S"], c["H"], c["dh"], dtype=torch.bfloat16, device=dev)
    o_view = out.permute(0, 2, 1, 3)
    row_ptr, entries, order, n_lead = _device_work_list(c["S"], c["window"], c["n_persistent"],
                                                        True, pattern, block_size, dev)
    import ctypes
    st = lambda t: (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))  # noqa: E731
    L = _lib.lib()
    stream = _lib.stream_ptr(dev)
    args = (_lib.ptr(q), st(q), _lib.ptr(k), st(k), _lib.ptr(v), st(v), _lib.ptr(out), st(o_view),
            None, c["B"], c["H"], c["S"], c["dh"], c["window"], c["n_persistent"], 1,
            pattern, block_size, float(1.0 / np.sqrt(c["dh"])), _lib.ptr(row_ptr),
            _lib.ptr(entries), _lib.ptr(order), n_lead, _lib.BF16, stream)

    def launch():
        rc = L.tmac_wattn_fwd(*args)
        if rc:
            _lib.check(rc, "tmac_wattn_fwd")

    if pattern == _lib.PATTERN_BAND:
        pairs = band_pairs(c["S"], c["window"], c["n_persistent"])
    else:  # allowed pairs from the host's per-row intervals
        rows = np.zeros(3 * c["S"], dtype=np.int32)
        cols = np.zeros(3 * c["S"], dtype=np.int32)
        _lib.check(L.tmac_wattn_mask_spans(c["S"], c["window"], c["n_persistent"], 1, pattern,
                                           block_size, rows.ctypes.data, cols.ctypes.data), "spans")
        np_, lo, hi = rows.reshape(-1, 3).T.astype(np.int64)
        pairs = int(np.sum(np_ + np.maximum(0, hi - np.maximum(lo, np_) + 1)))
    bh = c["B"] * c["H"]
    flops = 4 * c["dh"] * pairs * bh
    bytes_ = 4 * bh * c["S"] * c["dh"] * 2
    return dict(launch=launch, flops=flops, bytes=bytes_, tokens=c["B"] * c["S"],
                keep=(qkv, out, row_ptr, entries, order), q=q, k=k, v=v, fwd_args=args)


def setup_attn_cfg1(dev):
    """Config 1 on the GPU: the fp32 WindowedAttention module (qkv GEMM -> fp32 tile
    kernel -> out GEMM) at B=2, T=512, d=512, 8 heads, w=256, Np=16, eval, the shape
    cpu_secondary times on the host."""
    from titans_core.attn.windowed_attention import WindowConfig, WindowedAttention
    torch.manual_seed(1)
    B1, T1, d1, H1 = 2, 512, 512, 8
    mod = WindowedAttention(WindowConfig(window_size=256, num_heads=H1, head_dim=d1 // H1,
                                         n_persistent=16)).to(dev).eval()
    x = gen((B1, T1, d1), 1, dtype=torch.float32).to(dev)
    xg = x.clone().requires_grad_(True)
    gy = gen((B1, T1, d1), 2, dtype=torch.float32).to(dev)

    def launch():
        with torch.no_grad():
            mod(x)

    def train():  # forward + backward (input and weight gradients)
        mod(xg).backward(gy)

    return dict(launch=launch, train=train, tokens=B1 * T1, keep=(mod, x, xg, gy))


def setup_attn_bwd(dev, att):
    """Backward of the config-3 attention (dQ, dK, dV from dO) on the forward's views."""
    import ctypes
    c = CFG3
    B, H, S, dh = c["B"], c["H"], c["S"], c["dh"]
    q, k, v = att["q"], att["k"], att["v"]
    scale = float(1.0 / np.sqrt(dh))
    out, lse = window_attn_fwd(q, k, v, c["window"], c["n_persistent"], True, _lib.PATTERN_BAND,
                               64, scale, True)
    do = gen((B, S, H, dh), c["seed"] + 1).to(dev)
    grads = [torch.empty(B, S, H, dh, dtype=torch.bfloat16, device=dev) for _ in range(3)]
    delta = torch.empty(B, H, S, dtype=torch.float32, device=dev)
    row_ptr, entries, order, n_lead = _device_work_list(S, c["window"], c["n_persistent"], True,
                                                        _lib.PATTERN_BAND, 64, dev)
    col_ptr, entries_kv, order_kv, n_lead_kv = _device_work_list_kv(
        S, c["window"], c["n_persistent"], True, _lib.PATTERN_BAND, 64, dev)
    st = lambda t: (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))  # noqa: E731
    pv = lambda t: st(t.permute(0, 2, 1, 3))  # noqa: E731  [B, S, H, dh] buffer as [B, H, S, dh]
    L = _lib.lib()
    args = (_lib.ptr(q), st(q), _lib.ptr(k), st(k), _lib.ptr(v), st(v), _lib.ptr(out), pv(out),
            _lib.ptr(do), pv(do), _lib.ptr(lse), _lib.ptr(delta),
            _lib.ptr(grads[0]), pv(grads[0]), _lib.ptr(grads[1]), pv(grads[1]),
            _lib.ptr(grads[2]), pv(grads[2]), B, H, S, dh, c["window"], c["n_persistent"], 1,
            _lib.PATTERN_BAND, 64, scale, _lib.ptr(row_ptr), _lib.ptr(entries), _lib.ptr(order),
            n_lead, _lib.ptr(col_ptr), _lib.ptr(entries_kv), _lib.ptr(order_kv), n_lead_kv,
            _lib.BF16, _lib.stream_ptr(dev))

    def launch():
        rc = L.tmac_wattn_bwd(*args)
        if rc:
            _lib.check(rc, "tmac_wattn_bwd")

    pairs = band_pairs(S, c["window"], c["n_persistent"])
    flops = 10 * dh * pairs * B * H  # dS·K, dSᵀ·Q, Pᵀ·dO, dO·Vᵀ, Q·Kᵀ: 5 products of 2·dh per pair
    return dict(launch=launch, flops=flops, tokens=B * S, do=do, out=out, bwd_args=args,
                keep=(out, lse, do, grads, delta, row_ptr, entries, order, col_ptr, entries_kv,
                      order_kv))


def setup_attn_ex(dev, att, bwd, mask: bool, dropout_p: float):
    """Config-3 attention through tmac_wattn_fwd_ex / _bwd_ex: the band mask passed as a
    caller's bool [S, S] tensor (mask=True, work lists built on the device by
    tmac_wattn_mask_lists) and/or attention dropout. Returns fwd and bwd launches and the
    mask-list build launch."""
    import ctypes
    from titans_core.kernels.window_attn import AttnOpts
    from titans_core.attn.windowed_attention import build_band_mask
    c = CFG3
    B, H, S, dh = c["B"], c["H"], c["S"], c["dh"]
    L = _lib.lib()
    o = AttnOpts()
    o.dropout_p = dropout_p
    o.dropout_seed = 12345
    keep = []
    if mask:
        m = build_band_mask(S, c["window"], c["n_persistent"], str(dev)).view(torch.uint8)
        ws = torch.empty(L.tmac_wattn_mask_workspace(S, 1, 1), dtype=torch.uint8, device=dev)
        o.d_mask, o.mask_format, o.mask_batch, o.mask_heads = m.data_ptr(), 0, 1, 1
        o.mask_strides[2] = m.stride(0)
        o.d_mask_ws, o.mask_ws_bytes = ws.data_ptr(), ws.numel()
        keep += [m, ws]
    stream = _lib.stream_ptr(dev)

    def lists():
        rc = L.tmac_wattn_mask_lists(ctypes.byref(o), S, stream)
        if rc:
            _lib.check(rc, "tmac_wattn_mask_lists")

    if mask:
        lists()
    fa = att["fwd_args"]
    ba = bwd["bwd_args"]

    def fwd():
        rc = L.tmac_wattn_fwd_ex(*fa, ctypes.byref(o))
        if rc:
            _lib.check(rc, "tmac_wattn_fwd_ex")

    def bwd_launch():
        rc = L.tmac_wattn_bwd_ex(*ba, ctypes.byref(o))
        if rc:
            _lib.check(rc, "tmac_wattn_bwd_ex")

    return dict(fwd=fwd, bwd=bwd_launch, lists=lists if mask else None, keep=(keep, o))


def dense_attention_bwd_baseline(att, bwd, steps: int, stream):
    """ms of the dense masked backward in bf16 on this GPU, the products autograd of the
    reference's masked SDPA runs: softmax(Q·Kᵀ·scale + mask) recomputed, then dV, dP, dQ
    and dK as bmm over the full S x S (every transposed operand made contiguous first)."""
    c = CFG3
    B, H, S, dh = c["B"], c["H"], c["S"], c["dh"]
    i = torch.arange(S, device=att["q"].device)
    j = i[None, :]
    i = i[:, None]
    Np, w = c["n_persistent"], c["window"]
    allowed = (j < Np) | ((i >= Np) & (j >= Np) & (j >= i - w) & (j <= i))
    add = torch.zeros(S, S, dtype=torch.bfloat16, device=i.device).masked_fill(~allowed, float("-inf"))
    qb = att["q"].reshape(B * H, S, dh).contiguous()
    kb = att["k"].reshape(B * H, S, dh).contiguous()
    vb = att["v"].reshape(B * H, S, dh).contiguous()
    kt, vt = kb.transpose(1, 2).contiguous(), vb.transpose(1, 2).contiguous()
    dob = bwd["do"].permute(0, 2, 1, 3).reshape(B * H, S, dh).contiguous()
    ob = bwd["out"].permute(0, 2, 1, 3).reshape(B * H, S, dh).contiguous()
    scale = 1.0 / dh ** 0.5

    def dense_bwd():
        p = torch.softmax(torch.bmm(qb, kt) * scale + add, dim=-1)
        dv = torch.bmm(p.transpose(1, 2).contiguous(), dob)
        dp = torch.bmm(dob, vt)
        ds = p * (dp - (dob * ob).sum(-1, keepdim=True))
        dq = torch.bmm(ds, kb) * scale
        dk = torch.bmm(ds.transpose(1, 2).contiguous(), qb) * scale
        return dq, dk, dv

    return timed(dense_bwd, max(2, steps // 10), 2, stream)


CFG5 = dict(B=4, T=4096, vocab_size=50000, d_model=640, n_heads=10, n_layers=16, window_size=512,
            n_persistent=16, seed=7)


def setup_mac(dev, test_time_memory=False, graph=False):
    """Config 5: TitanMAC forward (MAC) with the Block-ELL MLP at 50%, bf16, eval; with graph,
    the layer stack of each segment replays a captured HIP graph (TitanMAC.capture_block_graph)."""
    sys.path.insert(0, str(ROOT / "titanmac-standalone_amd"))
    import titans_core as tc
    c = CFG5
    cfg = tc.TitanMACConfig(vocab_size=c["vocab_size"], d_model=c["d_model"], n_heads=c["n_heads"],
                            n_layers=c["n_layers"], window_size=c["window_size"],
                            n_persistent=c["n_persistent"], use_neural_memory=True,
                            titans_variant="MAC", memory_capacity=256, mlp_block_ell=True,
                            mlp_density=0.5, enable_test_time_memory=test_time_memory)
    torch.manual_seed(c["seed"])
    model = tc.TitanMAC(cfg).to(dev, torch.bfloat16).eval()
    if graph:
        model.capture_block_graph(c["B"])
    g = torch.Generator().manual_seed(c["seed"] + 1)
    ids = torch.randint(0, c["vocab_size"], (c["B"], c["T"]), generator=g).to(dev)
    res = {}

    def launch():
        with torch.no_grad():
            res["out"] = model(ids)

    return dict(launch=launch, tokens=c["B"] * c["T"], keep=(model, ids, res))


def setup_memupd(dev):
    """The neural-memory update step (tmac_mem_update: norm, clip, momentum, forgetting) over
    config 5's memory MLP parameters, fp32, called through the C ABI with prebuilt arguments."""
    import ctypes
    d = CFG5["d_model"]
    sizes = [d * d, d, d * d, d]
    g = [gen((n,), 40 + i, 0.001, torch.float32).to(dev) for i, n in enumerate(sizes)]
    s_ = [gen((n,), 50 + i, 0.01, torch.float32).to(dev) for i, n in enumerate(sizes)]
    w = [gen((n,), 60 + i, 0.02, torch.float32).to(dev) for i, n in enumerate(sizes)]
    a = torch.tensor(0.01, device=dev)
    e = torch.tensor(0.9, device=dev)
    stats = torch.empty(4, dtype=torch.float32, device=dev)
    L = _lib.lib()
    n_t = len(sizes)
    sz = (ctypes.c_int64 * n_t)(*sizes)
    wsb = ctypes.c_size_t(0)
    _lib.check(L.tmac_mem_update_workspace(sz, n_t, ctypes.byref(wsb)), "workspace")
    ws = torch.empty(wsb.value, dtype=torch.uint8, device=dev)
    arr = lambda ts: (ctypes.c_void_p * n_t)(*[t.data_ptr() for t in ts])  # noqa: E731
    args = (arr(g), arr(s_), arr(w), None, sz, n_t, _lib.ptr(a), _lib.ptr(e), None,
            ctypes.c_float(1e-6), ctypes.c_float(1.0), _lib.MEM_CLIP_MEMORY, _lib.ptr(stats),
            _lib.ptr(ws), ws.numel(), _lib.F32, _lib.stream_ptr(dev))

    def launch():
        rc = L.tmac_mem_update(*args)
        if rc:
            _lib.check(rc, "tmac_mem_update")

    n = sum(sizes)
    return dict(launch=launch, params=n, bytes=20 * n, keep=(g, s_, w, a, e, stats, ws, args))


CONV = dict(B=8, T=4096, C=1920, k=4, seed=5)   # BlockSparseAttention q/k/v conv at config 3's shape
NORM = dict(M=32768, D=640, seed=6)               # TitanBlock RMSNorm over config 3's tokens


def setup_conv(dev):
    """Causal depthwise conv (fused q/k/v channels) forward and backward, bf16."""
    import ctypes
    c = CONV
    B, T, C, k = c["B"], c["T"], c["C"], c["k"]
    x = gen((B, T, C), c["seed"]).to(dev)
    w = gen((C, k), c["seed"] + 1, 0.5).to(dev)
    dy = gen((B, T, C), c["seed"] + 2).to(dev)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    dw = torch.empty(C, k, dtype=torch.float32, device=dev)
    L = _lib.lib()
    n = ctypes.c_size_t(0)
    _lib.check(L.tmac_dwconv_causal_bwd_workspace(B, T, C, k, ctypes.byref(n)), "workspace")
    ws = torch.empty(n.value, dtype=torch.uint8, device=dev)
    stream = _lib.stream_ptr(dev)

    def fwd():
        rc = L.tmac_dwconv_causal(_lib.ptr(x), C, _lib.ptr(w), _lib.ptr(y), C, B, T, C, k,
                                  _lib.BF16, stream)
        if rc:
            _lib.check(rc, "tmac_dwconv_causal")

    def bwd():
        rc = L.tmac_dwconv_causal_bwd(_lib.ptr(dy), C, _lib.ptr(x), C, _lib.ptr(w), _lib.ptr(dx),
                                      C, _lib.ptr(dw), _lib.ptr(ws), ws.numel(), B, T, C, k,
                                      _lib.BF16, stream)
        if rc:
            _lib.check(rc, "tmac_dwconv_causal_bwd")

    act = B * T * C * 2
    return dict(fwd=fwd, bwd=bwd, fwd_bytes=2 * act, bwd_bytes=3 * act,
                keep=(x, w, dy, y, dx, dw, ws))


def setup_norm(dev):
    """RMSNorm forward and backward, bf16 [M, D]."""
    import ctypes
    c = NORM
    M, D = c["M"], c["D"]
    x = gen((M, D), c["seed"]).to(dev)
    sc = gen((D,), c["seed"] + 1).to(dev)
    dy = gen((M, D), c["seed"] + 2).to(dev)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    rstd = torch.empty(M, dtype=torch.float32, device=dev)
    dsc = torch.empty(D, dtype=torch.float32, device=dev)
    L = _lib.lib()
    n = ctypes.c_size_t(0)
    _lib.check(L.tmac_rmsnorm_bwd_workspace(M, D, ctypes.byref(n)), "workspace")
    ws = torch.empty(n.value, dtype=torch.uint8, device=dev)
    stream = _lib.stream_ptr(dev)

    def fwd():
        rc = L.tmac_rmsnorm_fwd(_lib.ptr(x), D, _lib.ptr(sc), _lib.ptr(y), D, _lib.ptr(rstd), M, D,
                                1e-5, _lib.BF16, stream)
        if rc:
            _lib.check(rc, "tmac_rmsnorm_fwd")

    def bwd():
        rc = L.tmac_rmsnorm_bwd(_lib.ptr(dy), D, _lib.ptr(x), D, _lib.ptr(sc), _lib.ptr(rstd),
                                _lib.ptr(dx), D, _lib.ptr(dsc), _lib.ptr(ws), ws.numel(), M, D,
                                _lib.BF16, stream)
        if rc:
            _lib.check(rc, "tmac_rmsnorm_bwd")

    fwd()
    act = M * D * 2
    return dict(fwd=fwd, bwd=bwd, fwd_bytes=2 * act + 4 * M, bwd_bytes=3 * act + 4 * M,
                keep=(x, sc, dy, y, dx, rstd, dsc, ws))


def setup_dx_sddmm(dev):
    c = CFG4
    pat = BlockELLPattern.sample(c["seed"], c["n_brow"], c["n_bcol"], c["width"])
    K, N, M = BS * c["n_brow"], BS * c["n_bcol"], c["M"]
    X = gen((M, K), c["seed"] + 1).to(dev)
    dY = gen((M, N), c["seed"] + 2).to(dev)
    V = gen((c["n_brow"], c["width"], BS, BS), c["seed"] + 3, 0.02).to(dev)
    dX = torch.empty(M, K, dtype=torch.bfloat16, device=dev)
    dV = torch.empty(c["n_brow"], c["width"], BS, BS, dtype=torch.float32, device=dev)
    idx = pat.device_index(dev)
    L = _lib.lib()
    ws_bytes = _sddmm_workspace_bytes(L, M, c["n_brow"], c["n_bcol"], c["width"])
    ws = torch.empty(ws_bytes // 4 + 4, dtype=torch.float32, device=dev)
    stream = _lib.stream_ptr(dev)
    dx_args = (_lib.ptr(dY), N, _lib.ptr(V), _lib.ptr(idx["col_idx"]), _lib.ptr(dX), K, M,
               c["n_brow"], c["n_bcol"], c["width"], _lib.BF16, stream)
    sd_args = (_lib.ptr(X), K, _lib.ptr(dY), N, _lib.ptr(idx["col_idx"]), _lib.ptr(dV), _lib.F32,
               _lib.ptr(ws), ws.numel() * 4, M, c["n_brow"], c["n_bcol"], c["width"], _lib.BF16,
               stream)

    def launch_dx():
        rc = L.tmac_bell_dx(*dx_args)
        if rc:
            _lib.check(rc, "tmac_bell_dx")

    def launch_sddmm():
        rc = L.tmac_bell_sddmm(*sd_args)
        if rc:
            _lib.check(rc, "tmac_bell_sddmm")

    nnz = c["n_brow"] * c["width"]
    flops = 2 * M * nnz * BS * BS
    dx_bytes = M * N * 2 + nnz * BS * BS * 2 + M * K * 2
    sd_bytes = M * K * 2 + M * N * 2 + nnz * BS * BS * 4
    return dict(dx=launch_dx, sddmm=launch_sddmm, flops=flops, dx_bytes=dx_bytes,
                sd_bytes=sd_bytes, keep=(X, dY, V, dX, dV, ws, idx))


def dense_attention_baseline(att, steps: int, warmup: int, stream):
    """ms of the reference's dense path on this GPU: masked SDPA, and bmm -> softmax -> bmm."""
    c = CFG3
    S = c["S"]
    i = torch.arange(S, device=att["q"].device)
    j = i[None, :]
    i = i[:, None]
    Np, w = c["n_persistent"], c["window"]
    allowed = (j < Np) | ((i >= Np) & (j >= Np) & (j >= i - w) & (j <= i))
    add = torch.zeros(S, S, dtype=torch.bfloat16, device=i.device).masked_fill(~allowed, float("-inf"))
    q, k, v = att["q"], att["k"], att["v"]
    res = {}
    sdpa = lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=add)  # noqa: E731
    res["sdpa_masked_ms"] = timed(sdpa, max(2, steps // 10), 2, stream)
    B, H, dh = c["B"], c["H"], c["dh"]
    qb = q.reshape(B * H, S, dh)
    kt = k.reshape(B * H, S, dh).transpose(1, 2).contiguous()
    vb = v.reshape(B * H, S, dh)

    def bmm_path():
        s = torch.bmm(qb, kt) * (1.0 / dh ** 0.5) + add
        return torch.bmm(torch.softmax(s, dim=-1), vb)

    res["bmm_softmax_bmm_ms"] = timed(bmm_path, max(2, steps // 10), 2, stream)
    return res


def dense_gemm_baseline(spmm, dev, steps: int, stream) -> float:
    """ms of the dense bf16 GEMM the reference's MLP runs for the same layer (nn.Linear:
    X[8192, 2560] @ W[2560, 10240] with the zero blocks stored), hipBLASLt through torch."""
    sys.path.insert(0, str(ROOT))
    c = CFG2
    W = torch.zeros(BS * c["n_brow"], BS * c["n_bcol"], dtype=torch.bfloat16)
    ci = spmm["pat"].col_idx
    for r in range(c["n_brow"]):
        for s_, col in enumerate(ci[r].tolist()):
            W[BS * r:BS * r + BS, BS * col:BS * col + BS] = spmm["V_cpu"][r, s_]
    X, Wd = spmm["X_cpu"].to(dev), W.to(dev)
    Y = torch.empty(X.shape[0], Wd.shape[1], dtype=torch.bfloat16, device=dev)
    return timed(lambda: torch.mm(X, Wd, out=Y), max(2, steps // 2), 3, stream)


def cpu_threads() -> tuple[int, dict]:
    """Threads for the CPU baselines and what the host reports. The GPU box gives each
    one-GPU job a share of its CPUs and presets OMP_NUM_THREADS to that share (16);
    threads beyond it would only oversubscribe cores that other jobs hold, so the
    baselines use min(CPUs in this process's affinity mask, OMP_NUM_THREADS)."""
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS")
    n = min(affinity, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else affinity
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    info = {"os_cpu_count": os.cpu_count(), "affinity_cpus": affinity, "omp_num_threads_env": omp,
            "cpu_model": model, **cpu_topology()}
    return max(1, n), info


def cpu_topology() -> dict:
    """Physical cores and hardware threads behind this process's CPUs (sysfs topology),
    and the clocks the host reports, so that a per-thread rate can be checked against a
    core's peak: SMT siblings share one core's FMA units."""
    cpus = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    cores, pkgs = set(), set()
    for c in cpus:
        base = Path(f"/sys/devices/system/cpu/cpu{c}/topology")
        try:
            pkg = int((base / "physical_package_id").read_text())
            core = int((base / "core_id").read_text())
        except (OSError, ValueError):
            return {"physical_cores": None, "threads_per_core": None, "cpu_mhz": None}
        cores.add((pkg, core))
        pkgs.add(pkg)
    mhz = []
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("cpu mhz"):
                mhz.append(float(line.split(":", 1)[1]))
    except (OSError, ValueError):
        pass
    max_mhz = None
    try:
        max_mhz = int(Path("/sys/devices/system/cpu/cpu0/cpufreq/cpuinfo_max_freq").read_text()) / 1000
    except (OSError, ValueError):
        pass
    return {"physical_cores": len(cores), "sockets": len(pkgs),
            "threads_per_core": round(len(cpus) / max(1, len(cores)), 2),
            "cpu_mhz": round(float(np.median(mhz)), 1) if mhz else None, "cpu_max_mhz": max_mhz}


def cpu_baseline(spmm) -> dict:
    """The oracle's dense restatement of config 2 (fp32 numpy X @ to_dense(W), the
    reference's nn.Linear with the zero blocks stored) on the host cores: a 2048-row
    sample for about 10 s, effective (stored-block) FLOPs counted as on the GPU."""
    sys.path.insert(0, str(ROOT))
    from oracle import block_ell as ob  # the checker / CPU baseline only
    from threadpoolctl import threadpool_info, threadpool_limits
    c = CFG2
    n, info = cpu_threads()
    X = spmm["X_cpu"].float().numpy()
    W = ob.to_dense(spmm["pat"].col_idx, spmm["V_cpu"].float().numpy(), c["n_bcol"])
    rows = 2048
    Xs = np.ascontiguousarray(X[:rows])
    with threadpool_limits(limits=n, user_api="blas"):
        blas = [p for p in threadpool_info() if p.get("user_api") == "blas"]
        blas_threads = max([p.get("num_threads", 0) for p in blas] or [0])
        _ = Xs @ W
        reps, t0 = 0, time.perf_counter()
        while True:
            _ = Xs @ W
            reps += 1
            el = time.perf_counter() - t0
            if el > 10.0:
                break
    eff = 2 * rows * c["n_brow"] * c["width"] * BS * BS
    dense = 2 * rows * BS * c["n_brow"] * BS * c["n_bcol"]
    return {"value": round(eff * reps / el / 1e12, 4), "unit": "TFLOP/s", "cores": int(blas_threads),
            "kind": "port",
            "sample": f"oracle dense fp32 X[{rows},2560] @ to_dense(W)[2560,10240] (numpy, "
                      f"{blas[0].get('internal_api') if blas else '?'} BLAS), {reps} reps in {el:.1f} s; "
                      f"effective (stored-block) FLOPs counted, as on the GPU",
            "dense_gflops_per_thread": round(dense * reps / el / 1e9 / max(1, blas_threads), 1),
            "dense_gflops_per_physical_core": round(
                dense * reps / el / 1e9 / max(1, min(blas_threads, info.get("physical_cores") or blas_threads)), 1),
            "torch_threads": torch.get_num_threads(), "blas_threads": blas_threads, **info}


def cpu_secondary() -> dict:
    """CPU timings of the reference-equivalent PyTorch paths of configs 1, 3 and 4 (fp32,
    torch on the host, the same threads as cpu_baseline): the WindowedAttention module
    (qkv GEMM -> SDPA with the additive [S, S] band mask -> out GEMM), the dense masked
    SDPA of config 3, and the dense-equivalent dX of config 4 on a row sample."""
    n, _ = cpu_threads()
    old = torch.get_num_threads()
    torch.set_num_threads(n)
    F = torch.nn.functional
    from titans_core.attn.windowed_attention import build_band_mask
    res = {}
    try:
        def med(fn, reps):
            fn()
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
            return float(np.median(ts))

        g = torch.Generator().manual_seed(1)
        # config 1: B=2, T=512, d=512, H=8, w=256, Np=16 (persistent tokens part of the sequence)
        B1, T1, d1, H1 = 2, 512, 512, 8
        x = torch.randn(B1, T1, d1, generator=g)
        wqkv = torch.randn(3 * d1, d1, generator=g) * 0.02
        wout = torch.randn(d1, d1, generator=g) * 0.02
        add1 = torch.zeros(T1, T1).masked_fill(~build_band_mask(T1, 256, 16, "cpu", True),
                                               float("-inf"))

        def cfg1():
            q, k, v = F.linear(x, wqkv).chunk(3, dim=-1)
            q, k, v = (t.reshape(B1, T1, H1, -1).transpose(1, 2) for t in (q, k, v))
            o = F.scaled_dot_product_attention(q, k, v, attn_mask=add1)
            return F.linear(o.transpose(1, 2).reshape(B1, T1, d1), wout)

        t1 = med(cfg1, 20)
        res["cfg1_windowed_attention_module_fp32_ms"] = round(t1 * 1e3, 3)
        res["cfg1_tokens_per_s"] = round(B1 * T1 / t1, 1)
        # config 3: dense masked SDPA, B=8, H=10, S=4096, dh=64 (343.6 GFLOP per call)
        c = CFG3
        S = c["S"]
        q3, k3, v3 = (torch.randn(c["B"], c["H"], S, c["dh"], generator=g) for _ in range(3))
        add3 = torch.zeros(S, S).masked_fill(~build_band_mask(S, c["window"], c["n_persistent"], "cpu",
                                                              True), float("-inf"))
        t3 = med(lambda: F.scaled_dot_product_attention(q3, k3, v3, attn_mask=add3), 2)
        res["cfg3_dense_masked_sdpa_fp32_ms"] = round(t3 * 1e3, 1)
        res["cfg3_tokens_per_s"] = round(c["B"] * S / t3, 1)
        del q3, k3, v3, add3
        # config 4: dX = dY . W^T dense-equivalent, 4096-row sample of dY [32768, 2560]
        c4 = CFG4
        dy = torch.randn(4096, BS * c4["n_bcol"], generator=g)
        w4 = torch.randn(BS * c4["n_brow"], BS * c4["n_bcol"], generator=g)
        t4 = med(lambda: dy @ w4.T, 10)
        eff4 = 2 * 4096 * c4["n_brow"] * c4["width"] * BS * BS
        res["cfg4_dx_dense_fp32_effective_tflops"] = round(eff4 / t4 / 1e12, 4)
        res["threads"] = torch.get_num_threads()
    finally:
        torch.set_num_threads(old)
    return res


def measure_traffic(timeout_s: int = 150) -> dict | None:
    """HBM bytes per launch of the config-2 SpMM forward, measured now on the current
    build: two rocprofv3 counter runs (FETCH_SIZE, then WRITE_SIZE) of `bench.py --mode
    traffic`, which launches a plain 1 GiB device copy and the SpMM kernel; each counter is
    scaled by what it reads for the copy of known size. None (with a message on stderr)
    when rocprofv3 is unavailable or a run fails."""
    import csv
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3")
    if not prof:
        print("bench.py: rocprofv3 not found; roofline.traffic is null", file=sys.stderr)
        return None
    vals = {}
    with tempfile.TemporaryDirectory(prefix="tmac_traffic_") as tmp:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            d = Path(tmp) / counter
            cmd = ["timeout", "-s", "KILL", str(timeout_s), prof, "--pmc", counter, "-f", "csv",
                   "-d", str(d), "-o", "run", "--", sys.executable, str(ROOT / "bench.py"),
                   "--mode", "traffic"]
            r = subprocess.run(cmd, capture_output=True, text=True, cwd=ROOT)
            files = sorted(d.rglob("*counter_collection.csv"))
            if r.returncode != 0 and not files:
                print(f"bench.py: rocprofv3 {counter} run failed (rc {r.returncode}); "
                      f"roofline.traffic is null\n{r.stderr[-1000:]}", file=sys.stderr)
                return None
            rows = [row for f in files for row in csv.DictReader(open(f))]
            # the runtime splits each 1 GiB copy into several dispatches: the copy's figure
            # is the sum over its dispatches per copy; the SpMM is one dispatch per launch
            for kind, sub in (("copy", "copyBuffer"), ("spmm", "bell_")):
                v = [float(row["Counter_Value"]) for row in rows
                     if sub in row.get("Kernel_Name", "") and row.get("Counter_Name") == counter]
                if not v:
                    print(f"bench.py: no {counter} samples for {kind}; roofline.traffic is null",
                          file=sys.stderr)
                    return None
                vals[(kind, counter)] = sum(v) / TRAFFIC_REPS if kind == "copy" else float(np.mean(v))
    gib_kib = float(1 << 20)  # the copy reads and writes 1 GiB = 1,048,576 KiB
    f_fetch = gib_kib / vals[("copy", "FETCH_SIZE")]
    f_write = gib_kib / vals[("copy", "WRITE_SIZE")]
    rd = vals[("spmm", "FETCH_SIZE")] * f_fetch * 1024
    wr = vals[("spmm", "WRITE_SIZE")] * f_write * 1024
    return {"traffic_bytes": rd + wr, "read_bytes": rd, "write_bytes": wr,
            "fetch_scale": f_fetch, "write_scale": f_write,
            "spmm_FETCH_SIZE_KiB": vals[("spmm", "FETCH_SIZE")],
            "spmm_WRITE_SIZE_KiB": vals[("spmm", "WRITE_SIZE")]}


def main() -> int:
    ap = argparse.ArgumentParser(description="TitanMAC sparse hot path benchmark (one MI355X)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-dense", action="store_true",
                    help="with --mode attn_bwd: skip the dense baseline (profiling runs)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 measurement of roofline.traffic (null)")
    ap.add_argument("--mode", default="all", choices=["all", "spmm", "attn", "attn_cfg1", "attn_bwd", "attn_ex", "dx",
                                                     "bell_f32", "mlp_train",
                                                     "sddmm", "conv",
                                                     "norm", "mac", "mac_ttm", "memupd", "copy",
                                                     "traffic"])
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the hot path's kernels run on one MI355X and this "
              "build has no multi-GPU code path; run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    K, W = args.steps, args.warmup

    if args.mode == "traffic":
        # what measure_traffic's counter runs see: a 1 GiB device copy, then the SpMM
        src = torch.empty(1 << 29, dtype=torch.int16, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(TRAFFIC_REPS):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        spmm = setup_spmm(dev)
        for _ in range(TRAFFIC_REPS):
            spmm["launch"]()
        torch.cuda.synchronize()
        print(json.dumps({"mode": "traffic", "done": True}))
        return 0

    if args.mode == "copy":
        src = torch.empty(1 << 29, dtype=torch.int16, device=dev).fill_(1)  # 1 GiB
        dst = torch.empty_like(src)
        ms = timed(lambda: dst.copy_(src), K, W, stream)
        print(json.dumps({"mode": "copy", "bytes_read": src.numel() * 2, "bytes_written": dst.numel() * 2,
                          "ms": ms, "GB/s": 2 * src.numel() * 2 / ms / 1e6}))
        return 0

    out = {}
    if args.mode in ("all", "spmm"):
        spmm = setup_spmm(dev)
        settle(spmm["launch"], CLOCK_SETTLE_S)
        ms = timed(spmm["launch"], K, W, stream)
        out["spmm"] = dict(ms=ms, tflops=spmm["flops"] / ms / 1e9, flops=spmm["flops"],
                           bytes=spmm["bytes"])
        if args.mode == "all":
            out["spmm"]["dense_ms"] = dense_gemm_baseline(spmm, dev, K, stream)
        out["spmm"]["gather_ms"] = timed(spmm["launch_gather"], K, W, stream)
        out["spmm"]["rr_ms"] = timed(spmm["launch_rr"], K, W, stream)
        out["spmm"]["m64_ms"] = timed(spmm["launch_m64"], K, W, stream)
        out["spmm"]["m64_weight_tbs"] = spmm["weight_bytes"] / out["spmm"]["m64_ms"] / 1e9
    if args.mode in ("all", "attn", "attn_bwd"):
        att = setup_attn(dev)
    if args.mode in ("all", "attn"):
        ms = timed(att["launch"], K, W, stream)
        out["attn"] = dict(ms=ms, tokens_per_s=att["tokens"] / ms * 1e3,
                           tflops=att["flops"] / ms / 1e9, gbs=att["bytes"] / ms / 1e6)
        if args.mode == "all":
            out["attn"].update(dense_attention_baseline(att, K, W, stream))
            for key, kw in (("s4112", dict(S=4112)),
                            ("blockwin", dict(pattern=_lib.PATTERN_BLOCKWIN))):
                extra = setup_attn(dev, **kw)
                ms_x = timed(extra["launch"], K, W, stream)
                out["attn"][key] = dict(ms=ms_x, tokens_per_s=extra["tokens"] / ms_x * 1e3,
                                        tflops=extra["flops"] / ms_x / 1e9)
                del extra
    if args.mode in ("all", "attn_cfg1"):
        wl = setup_attn_cfg1(dev)
        ms = timed(wl["launch"], K, W, stream)
        out["attn_cfg1"] = dict(ms=ms, tokens_per_s=wl["tokens"] / ms * 1e3,
                                train_ms=timed(wl["train"], K, W, stream))
        del wl
    if args.mode in ("all", "attn_bwd"):
        bwd = setup_attn_bwd(dev, att)
        ms = timed(bwd["launch"], K, W, stream)
        out["attn_bwd"] = dict(ms=ms, tokens_per_s=bwd["tokens"] / ms * 1e3,
                               tflops=bwd["flops"] / ms / 1e9)
        if not args.no_dense:
            out["attn_bwd"]["dense_bwd_ms"] = dense_attention_bwd_baseline(att, bwd, K, stream)
    if args.mode in ("all", "attn_ex"):
        if args.mode == "attn_ex":
            att = setup_attn(dev)
            bwd = setup_attn_bwd(dev, att)
        ex = {}
        for key, mask, p in (("mask", True, 0.0), ("dropout", False, 0.1),
                             ("mask_dropout", True, 0.1)):
            wl = setup_attn_ex(dev, att, bwd, mask, p)
            ex[key] = dict(fwd_ms=timed(wl["fwd"], K, W, stream),
                           bwd_ms=timed(wl["bwd"], K, W, stream))
            if wl["lists"] is not None and "lists_ms" not in ex:
                ex["lists_ms"] = timed(wl["lists"], K, W, stream)
            del wl
        out["attn_ex"] = ex
    if args.mode in ("all", "dx", "sddmm"):
        bw = setup_dx_sddmm(dev)
        if args.mode in ("all", "dx"):
            ms = timed(bw["dx"], K, W, stream)
            out["dx"] = dict(ms=ms, tflops=bw["flops"] / ms / 1e9, gbs=bw["dx_bytes"] / ms / 1e6)
        if args.mode in ("all", "sddmm"):
            ms = timed(bw["sddmm"], K, W, stream)
            out["sddmm"] = dict(ms=ms, tflops=bw["flops"] / ms / 1e9, gbs=bw["sd_bytes"] / ms / 1e6)

    if args.mode in ("all", "mlp_train"):
        wl = setup_mlp_train(dev)
        ms = timed(wl["launch"], K, W, stream)
        out["mlp_train"] = dict(ms=ms, tflops=wl["flops"] / ms / 1e9)
        del wl
    if args.mode in ("all", "bell_f32"):
        wl = setup_bell_f32(dev)
        f_ms = timed(wl["fwd"], K, W, stream)
        dx_ms = timed(wl["dx"], K, W, stream)
        sd_ms = timed(wl["sddmm"], K, W, stream)
        out["bell_f32"] = dict(fwd_ms=f_ms, fwd_tflops=wl["fwd_flops"] / f_ms / 1e9, dx_ms=dx_ms,
                               dx_tflops=wl["bwd_flops"] / dx_ms / 1e9, sddmm_ms=sd_ms,
                               sddmm_tflops=wl["bwd_flops"] / sd_ms / 1e9)
        del wl
    for mode, setup in (("conv", setup_conv), ("norm", setup_norm)):
        if args.mode in ("all", mode):
            wl = setup(dev)
            f_ms = timed(wl["fwd"], K, W, stream)
            b_ms = timed(wl["bwd"], K, W, stream)
            out[mode] = dict(fwd_ms=f_ms, fwd_gbs=wl["fwd_bytes"] / f_ms / 1e6, bwd_ms=b_ms,
                             bwd_gbs=wl["bwd_bytes"] / b_ms / 1e6)

    if args.mode in ("all", "memupd"):
        mu = setup_memupd(dev)
        ms = timed(mu["launch"], K, W, stream)
        out["memupd"] = dict(ms=ms, gbs=mu["bytes"] / ms / 1e6, params=mu["params"])
        del mu
    # whole-model forwards: a few steps keep the timed region to seconds
    k5, w5 = max(2, min(K, 10)), max(1, min(W, 3))
    for key, ttm, graph in (("mac", False, False), ("mac_ttm", True, False),
                            ("mac_ttm_graph", True, True)):
        if args.mode in ("all", key) or (key == "mac_ttm_graph" and args.mode == "mac_ttm"):
            wl = setup_mac(dev, ttm, graph)
            ms = timed(wl["launch"], k5, w5, stream)
            out[key] = dict(ms=ms, tokens_per_s=wl["tokens"] / ms * 1e3, steps=k5)
            del wl
            torch.cuda.empty_cache()

    if args.mode != "all":
        print(json.dumps({"mode": args.mode, **out}))
        return 0

    s = out["spmm"]
    a = out["attn"]
    dense_ms = min(a["sdpa_masked_ms"], a["bmm_softmax_bmm_ms"])
    tr = None if args.no_traffic else measure_traffic()
    traffic = None if tr is None else round(tr["traffic_bytes"])
    line = {
        "metric": METRIC,
        "value": round(s["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "clock_settle_s": CLOCK_SETTLE_S,
        "ms_per_step": round(s["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) block values, splitmix64 pattern)",
        "config": {"workload": "Block-ELL SpMM forward, BASELINE config 2: X[8192,2560] bf16 . "
                               "W[2560,10240] Block-ELL 64x64, width 40 of 160 (25%), fp32 "
                               "accumulate, bf16 out",
                   "M": CFG2["M"], "K": 2560, "N": 10240, "block": 64, "width": CFG2["width"],
                   "seed": CFG2["seed"]},
        "roofline": {"bound": "mfma", "achieved": round(s["tflops"], 3), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(s["tflops"] / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic},
        "secondary": {
            "dense_bf16_gemm_same_layer_ms": round(s["dense_ms"], 4),
            "spmm_speedup_vs_dense_gemm": round(s["dense_ms"] / s["ms"], 2),
            "windowed_attn_fwd_tokens_per_s": round(a["tokens_per_s"], 1),
            "windowed_attn_fwd_ms": round(a["ms"], 5),
            "windowed_attn_fwd_tflops_algorithmic": round(a["tflops"], 3),
            "windowed_attn_fwd_hbm_gbs_compulsory": round(a["gbs"], 1),
            "dense_masked_sdpa_ms": round(a["sdpa_masked_ms"], 4),
            "dense_bmm_softmax_bmm_ms": round(a["bmm_softmax_bmm_ms"], 4),
            "attn_speedup_vs_dense": round(dense_ms / a["ms"], 2),
            "windowed_attn_fwd_s4112_ms": round(a["s4112"]["ms"], 5),
            "windowed_attn_fwd_s4112_tokens_per_s": round(a["s4112"]["tokens_per_s"], 1),
            "blocksparse_attn_fwd_blockwin_ms": round(a["blockwin"]["ms"], 5),
            "blocksparse_attn_fwd_blockwin_tflops_algorithmic": round(a["blockwin"]["tflops"], 3),
            "windowed_attention_module_cfg1_fp32_ms": round(out["attn_cfg1"]["ms"], 5),
            "windowed_attention_module_cfg1_fp32_tokens_per_s": round(out["attn_cfg1"]["tokens_per_s"], 1),
            "windowed_attention_module_cfg1_fp32_fwd_bwd_ms": round(out["attn_cfg1"]["train_ms"], 5),
            "windowed_attn_bwd_ms": round(out["attn_bwd"]["ms"], 5),
            "windowed_attn_bwd_tflops_algorithmic": round(out["attn_bwd"]["tflops"], 3),
            "dense_masked_bwd_bmm_ms": round(out["attn_bwd"]["dense_bwd_ms"], 4),
            "attn_bwd_speedup_vs_dense": round(out["attn_bwd"]["dense_bwd_ms"] / out["attn_bwd"]["ms"], 2),
            "bell_fwd_cfg2_fp32_ms": round(out["bell_f32"]["fwd_ms"], 5),
            "bell_fwd_cfg2_fp32_tflops": round(out["bell_f32"]["fwd_tflops"], 2),
            "bell_dx_cfg4_fp32_ms": round(out["bell_f32"]["dx_ms"], 5),
            "bell_sddmm_cfg4_fp32_ms": round(out["bell_f32"]["sddmm_ms"], 5),
            "bell_fp32_peak_tflops": 157.3,
            "windowed_attn_fwd_caller_mask_ms": round(out["attn_ex"]["mask"]["fwd_ms"], 5),
            "windowed_attn_bwd_caller_mask_ms": round(out["attn_ex"]["mask"]["bwd_ms"], 5),
            "windowed_attn_mask_lists_us": round(out["attn_ex"]["lists_ms"] * 1e3, 2),
            "windowed_attn_fwd_dropout0.1_ms": round(out["attn_ex"]["dropout"]["fwd_ms"], 5),
            "windowed_attn_bwd_dropout0.1_ms": round(out["attn_ex"]["dropout"]["bwd_ms"], 5),
            "windowed_attn_fwd_mask_dropout0.1_ms": round(out["attn_ex"]["mask_dropout"]["fwd_ms"], 5),
            "windowed_attn_bwd_mask_dropout0.1_ms": round(out["attn_ex"]["mask_dropout"]["bwd_ms"], 5),
            "bell_fwd_cfg2_gather_kernel_ms": round(out["spmm"]["gather_ms"], 5),
            "bell_fwd_cfg2_grouped_round_robin_ms": round(out["spmm"]["rr_ms"], 5),
            "bell_fwd_cfg2_m64_us": round(out["spmm"]["m64_ms"] * 1e3, 2),
            "bell_fwd_cfg2_m64_weight_tbs": round(out["spmm"]["m64_weight_tbs"], 3),
            "bell_dx_cfg4_ms": round(out["dx"]["ms"], 5),
            "bell_dx_cfg4_tflops": round(out["dx"]["tflops"], 3),
            "bell_dx_cfg4_hbm_gbs_compulsory": round(out["dx"]["gbs"], 1),
            "bell_sddmm_cfg4_ms": round(out["sddmm"]["ms"], 5),
            "bell_sddmm_cfg4_tflops": round(out["sddmm"]["tflops"], 3),
            "bell_sddmm_cfg4_hbm_gbs_compulsory": round(out["sddmm"]["gbs"], 1),
            "bell_mlp_train_step_cfg4_ms": round(out["mlp_train"]["ms"], 5),
            "bell_mlp_train_step_cfg4_tflops": round(out["mlp_train"]["tflops"], 3),
            "dwconv_fwd_ms": round(out["conv"]["fwd_ms"], 5),
            "dwconv_fwd_hbm_gbs_compulsory": round(out["conv"]["fwd_gbs"], 1),
            "dwconv_bwd_ms": round(out["conv"]["bwd_ms"], 5),
            "dwconv_bwd_hbm_gbs_compulsory": round(out["conv"]["bwd_gbs"], 1),
            "rmsnorm_fwd_ms": round(out["norm"]["fwd_ms"], 5),
            "rmsnorm_fwd_hbm_gbs_compulsory": round(out["norm"]["fwd_gbs"], 1),
            "rmsnorm_bwd_ms": round(out["norm"]["bwd_ms"], 5),
            "rmsnorm_bwd_hbm_gbs_compulsory": round(out["norm"]["bwd_gbs"], 1),
            "titanmac_mac_fwd_cfg5_tokens_per_s": round(out["mac"]["tokens_per_s"], 1),
            "titanmac_mac_fwd_cfg5_ms": round(out["mac"]["ms"], 3),
            "titanmac_mac_fwd_cfg5_test_time_memory_tokens_per_s": round(
                out["mac_ttm"]["tokens_per_s"], 1),
            "titanmac_mac_fwd_cfg5_test_time_memory_ms": round(out["mac_ttm"]["ms"], 3),
            "titanmac_mac_fwd_cfg5_test_time_memory_block_graph_ms": round(out["mac_ttm_graph"]["ms"], 3),
            "neural_memory_update_cfg5_ms": round(out["memupd"]["ms"], 5),
            "neural_memory_update_cfg5_hbm_gbs_compulsory": round(out["memupd"]["gbs"], 1),
        },
    }
    if tr is not None:
        line["secondary"]["spmm_traffic_read_bytes"] = round(tr["read_bytes"])
        line["secondary"]["spmm_traffic_write_bytes"] = round(tr["write_bytes"])
        line["secondary"]["traffic_counter_scales"] = [round(tr["fetch_scale"], 4),
                                                       round(tr["write_scale"], 4)]
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(spmm)
        line["secondary"]["cpu"] = cpu_secondary()
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
