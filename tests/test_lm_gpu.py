"""Byte-level SSM LM on the GPU: embedding, RMSNorm, conv step, pre-norm
layers (prefill and decode) and the whole model, against the CPU oracle (oracle.lm_prefill /
oracle.lm_decode_step: f32 arithmetic with bf16 rounding at the device path's storage points).
Bars: embedding exact; RMSNorm fp32 1e-5 (rel_err); everything through a bf16 GEMM is held
normwise (max|g - r| / max|r|, see tests/test_block_gpu.py) at 1e-2 against the same-rounding
oracle. The decode path must continue a prefill: decoding token L after prefilling L tokens
matches the prefill of L + 1 tokens."""
import numpy as np
import pytest
import torch

import oracle
from helixml_amd import lm
from helixml_amd.lm import LAYER_KEYS, ByteLM
from tests.util import CW_ULPS, TOL_BF16, TOL_F32, bf16_round, block_inputs, cw_ulps, lm_params, norm_err, rel_err

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
BF_NAMES = {"w_in", "w_x", "w_dt", "w_out", "w_head"}


def to_dev(p, dev):
    return {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev, BF if k in BF_NAMES else torch.float32)
            for k, v in p.items()}


def model_from(P, dev, dt_rank, K=4, eps=1e-5):
    """A ByteLM whose weights are the given host parameters."""
    nl = len(P["layers"])
    dm = P["embed"].shape[1]
    di = P["layers"][0]["w_dt"].shape[0] if nl else 2 * dm
    m = ByteLM(n_layers=nl, d_model=dm, d_state=16, d_conv=K, expand=di // dm, dt_rank=dt_rank,
               vocab=P["embed"].shape[0], eps=eps, device=dev)
    m.embed = torch.from_numpy(P["embed"]).to(dev)
    m.norm_f = torch.from_numpy(P["norm_f"]).to(dev)
    m.w_head = torch.from_numpy(P["w_head"]).to(dev, BF)
    m.layers = [to_dev(p, dev) for p in P["layers"]]
    return m


def check_logits(g, ref, ref64, terms, what, norm_bar=1e-2):
    """Logits after bf16 GEMMs. Normwise against the same-rounding f32 oracle: within
    ``norm_bar``, or twice the f32 oracle's own normwise distance from its float64 twin (same
    rounding points) where that is larger. Elementwise against the float64 twin, componentwise:
    each logit within CW_ULPS bf16 ulps (2^-8) of ``terms`` = |xn| . |w_head|^T, the magnitudes
    of the terms that logit sums (a logit near zero is a cancellation, where the plain relative
    error measures the rounding of large terms against a small result; a few one-ulp flips of
    bf16 intermediates move a logit by a few ulps of its terms)."""
    e_norm, own_norm = norm_err(g, ref), norm_err(ref, ref64)
    e_cw, own_cw = cw_ulps(g, ref64, terms), cw_ulps(ref, ref64, terms)
    print(f"{what}: normwise {e_norm:.3e} (f32 oracle's own {own_norm:.3e}); componentwise {e_cw:.3f} bf16 "
          f"ulps of the terms (f32 oracle's own {own_cw:.3f}); plain elementwise {rel_err(g, ref64):.3e}",
          flush=True)
    assert e_norm <= max(norm_bar, 2 * own_norm), (what, e_norm, own_norm)
    assert e_cw <= CW_ULPS, (what, e_cw, own_cw)


def test_embedding_gather_and_invalid_tokens(dev):
    rng = np.random.default_rng(1)
    table = rng.standard_normal((256, 96)).astype(np.float32)
    tok = rng.integers(0, 256, (5, 33)).astype(np.int32)
    tok[0, 0], tok[1, 1] = -1, 256
    g = lm.embedding(torch.from_numpy(tok).to(dev), torch.from_numpy(table).to(dev)).cpu().numpy()
    ref = table[np.clip(tok, 0, 255)]
    ref[0, 0] = 0
    ref[1, 1] = 0
    assert np.array_equal(g, ref)


@pytest.mark.parametrize("rows,dim", [(7, 512), (130, 64), (3, 2048), (5, 100), (2, 3000)])
def test_rmsnorm(dev, rows, dim):
    rng = np.random.default_rng(rows + dim)
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float32)
    w = rng.standard_normal(dim).astype(np.float32)
    xd, wd = torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev)
    ref = oracle.rmsnorm(x, w, 1e-5)
    g = lm.rmsnorm(xd, wd, 1e-5).cpu().numpy()
    err = rel_err(g, ref)
    assert err < 1e-5, err
    gb = lm.rmsnorm(xd, wd, 1e-5, out_dtype=BF).float().cpu().numpy()
    err = rel_err(gb, bf16_round(ref))
    assert err <= 2.0 ** -7, err  # at most one bf16 ulp apart (rounding of nearly equal values)


@pytest.mark.parametrize("dtype", [torch.float32, BF])
@pytest.mark.parametrize("K", [4, 3, 2])
def test_conv1d_step_matches_full_conv(dev, dtype, K):
    rng = np.random.default_rng(K)
    bt, L, dim = 3, 12, 40
    x = bf16_round(rng.standard_normal((bt, L, 2 * dim)).astype(np.float32))
    w = rng.standard_normal((dim, K)).astype(np.float32)
    b = rng.standard_normal(dim).astype(np.float32)
    xd = torch.from_numpy(x).to(dev, dtype)
    wd, bd = torch.from_numpy(w).to(dev), torch.from_numpy(b).to(dev)
    state = torch.zeros((bt, K - 1, dim), device=dev)
    full = oracle.conv1d_silu(x[:, :, :dim], w, b)
    for t in range(L):
        y = lm.conv1d_step(xd[:, t, :dim], wd, bd, state).float().cpu().numpy()
        if dtype == torch.float32:
            err = rel_err(y, full[:, t])
            assert err < TOL_F32, (t, err)
        else:
            err = norm_err(y, full[:, t])
            assert err <= 2.0 ** -8, (t, err)
    # the state holds the last K-1 inputs
    want = x[:, L - (K - 1):, :dim].transpose(0, 1, 2)
    assert np.array_equal(state.cpu().numpy(), want.astype(np.float32))


def run_layer(dev, p, x, dt_rank, eps=1e-5):
    bt, L, dm = x.shape
    di = p["w_dt"].shape[0]
    K = p["conv_w"].shape[1]
    d = to_dev(p, dev)
    resid = torch.from_numpy(x).to(dev).contiguous()
    ssm_st = torch.zeros((bt, di, 16), device=dev)
    conv_st = torch.zeros((bt, K - 1, di), device=dev)
    need = int(lm._ffi.lib().hx_mamba_layer_workspace_size(bt, L, dm, di, dt_rank, 16))
    ws = torch.empty(need, device=dev, dtype=torch.uint8)
    lm._ffi.call("hx_mamba_layer_fwd", bt, L, dm, di, 16, dt_rank, K, resid.data_ptr(),
                 d["norm_w"].data_ptr(), eps, *[d[k].data_ptr() for k in LAYER_KEYS],
                 ssm_st.data_ptr(), conv_st.data_ptr(), ws.data_ptr(), need,
                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return resid.cpu().numpy(), ssm_st.cpu().numpy(), conv_st.cpu().numpy()


@pytest.mark.parametrize("bt,L,dm,di,r", [(2, 40, 64, 128, 8), (1, 130, 32, 64, 8), (3, 17, 48, 96, 16)])
def test_layer_prefill_and_state_handoff(dev, bt, L, dm, di, r):
    p = block_inputs(1, 1, dm, di, 16, r, 4, seed=bt + L)
    p.pop("x")
    p["norm_w"] = np.random.default_rng(L).uniform(0.5, 1.5, dm).astype(np.float32)
    x = np.random.default_rng(bt).standard_normal((bt, L, dm)).astype(np.float32)
    g, g_ssm, g_conv = run_layer(dev, p, x, r)
    xn = bf16_round(oracle.rmsnorm(x.reshape(-1, dm), p["norm_w"], 1e-5)).reshape(bt, L, dm)
    blk = {k: p[k] for k in LAYER_KEYS}
    out, last, conv = oracle.mamba_block(xn, **blk, dt_rank=r, round_out=False, return_state=True)
    ref = x + out
    err = norm_err(g - x, ref - x)
    assert err <= 1e-2, err
    err = norm_err(g_ssm, last)
    assert err <= 1e-2, err
    assert np.array_equal(g_conv, conv)  # the conv window is copied bf16 inputs


def test_lm_prefill_and_decode_vs_oracle(dev):
    P = lm_params(2, 64, 128, 16, 8, 4, 256, seed=5)
    m = model_from(P, dev, dt_rank=8)
    tok = np.random.default_rng(6).integers(0, 256, (3, 20)).astype(np.int32)
    td = torch.from_numpy(tok).to(dev)
    logits, state = m.prefill(td[:, :18])
    torch.cuda.synchronize()
    ref, rstate = oracle.lm_prefill(tok[:, :18], P, 8)
    ref64, rstate64, terms = oracle.numpy_lm_prefill(tok[:, :18], P, 8, return_terms=True)
    check_logits(logits.cpu().numpy(), ref, ref64, terms, "prefill")
    for t in (18, 19):
        lg = m.decode_step(td[:, t], state)
        torch.cuda.synchronize()
        rl, rstate = oracle.lm_decode_step(tok[:, t], P, rstate, 8)
        rl64, rstate64, terms = oracle.numpy_lm_decode_step(tok[:, t], P, rstate64, 8, return_terms=True)
        check_logits(lg.cpu().numpy(), rl, rl64, terms, f"decode step {t}")
    # decode continues the prefill: same logits as prefilling all 20 tokens
    full, _ = m.prefill(td)
    err = norm_err(lg.cpu().numpy(), full[:, 19].cpu().numpy())
    assert err <= 1e-2, err


@pytest.mark.parametrize("dm,di,r,K", [(640, 1280, 40, 4), (512, 1024, 64, 3)])
def test_lm_decode_general_shapes(dev, dm, di, r, K):
    """The fused decode step's general form: d_inner above 1024 (two pass-1 pairs and two pass-2
    rounds per thread, two x_proj channel blocks) with a dt_rank that is no multiple of 32 (element
    dt_proj loads), and dt_rank 64 (two x_proj output chunks, 16-byte dt_proj rows over two rank
    blocks) with a width-3 conv. Two decode steps against the oracle; decode continues the
    prefill."""
    P = lm_params(2, dm, di, 16, r, K, 256, seed=dm + r)
    m = model_from(P, dev, dt_rank=r, K=K)
    tok = np.random.default_rng(di).integers(0, 256, (3, 8)).astype(np.int32)
    td = torch.from_numpy(tok).to(dev)
    print(f"case decode d_model {dm} d_inner {di} dt_rank {r} conv {K}", flush=True)
    _, state = m.prefill(td[:, :6])
    _, rstate = oracle.lm_prefill(tok[:, :6], P, r)
    for t in (6, 7):
        lg = m.decode_step(td[:, t].contiguous(), state)
        torch.cuda.synchronize()
        rl, rstate = oracle.lm_decode_step(tok[:, t], P, rstate, r)
        err = norm_err(lg.cpu().numpy(), rl)
        assert err <= 1e-2, (t, err)
    full, _ = m.prefill(td)
    err = norm_err(lg.cpu().numpy(), full[:, 7].cpu().numpy())
    assert err <= 1e-2, err


@pytest.mark.parametrize("dm,di,r,K", [(132, 132, 12, 2), (100, 200, 16, 1), (1020, 1020, 32, 3),
                                       (512, 1024, 20, 4)])
def test_lm_decode_row_kernel_shapes(dev, dm, di, r, K):
    """The decode step's row kernel (d_inner <= 1024, dt_rank <= 32) off config 5's shape:
    8-byte W_x chunks (d_inner % 8 != 0: 132, 1020), 16-byte chunks with lanes past d_inner
    (200), conv widths 1 to 3, x_proj outputs past dt_rank + 32 on the last waves, element
    dt_proj rows (dt_rank 12, 16, 20) and the 16-byte ones (32). Two decode steps against the
    oracle; decode continues the prefill."""
    P = lm_params(2, dm, di, 16, r, K, 256, seed=di + r)
    m = model_from(P, dev, dt_rank=r, K=K)
    tok = np.random.default_rng(di + 1).integers(0, 256, (3, 8)).astype(np.int32)
    td = torch.from_numpy(tok).to(dev)
    print(f"case row decode d_model {dm} d_inner {di} dt_rank {r} conv {K}", flush=True)
    _, state = m.prefill(td[:, :6])
    _, rstate = oracle.lm_prefill(tok[:, :6], P, r)
    for t in (6, 7):
        lg = m.decode_step(td[:, t].contiguous(), state)
        torch.cuda.synchronize()
        rl, rstate = oracle.lm_decode_step(tok[:, t], P, rstate, r)
        err = norm_err(lg.cpu().numpy(), rl)
        assert err <= 1e-2, (t, err)
    full, _ = m.prefill(td)
    err = norm_err(lg.cpu().numpy(), full[:, 7].cpu().numpy())
    assert err <= 1e-2, err


@pytest.mark.parametrize("bt,dm,di", [(512, 256, 1024), (64, 256, 2560), (256, 512, 1024), (3, 64, 128)])
def test_lm_decode_fused_prenorm_tilings(dev, bt, dm, di):
    """The decode step's pre-norm folded into in_proj's operand load, in each tiling of the
    small-M GEMM it rides on: 64-wide tiles with 4 waves (batch 512, in_proj N 2048 K 256),
    32-wide with 4 waves (batch 64, N 5120), 64-wide with 8 waves (config 5's batch 256) and
    32-wide with 8 waves and two pieces per lane (batch 3, K 64). One decode step of a 1-layer
    model against the same step with the separate RMSNorm launch (a forced GEMM kernel takes the
    unfused form: the two differ only in the order of the rows' sums of squares, normwise <= 1e-3)
    and against the oracle on the first and last sequences."""
    from helixml_amd import ssm
    r = 16
    P = lm_params(1, dm, di, 16, r, 4, 256, seed=bt + di)
    m = model_from(P, dev, dt_rank=r)
    rng = np.random.default_rng(bt * 7 + dm)
    tok = rng.integers(0, 256, (bt, 5)).astype(np.int32)
    td = torch.from_numpy(tok).to(dev)
    print(f"case fused pre-norm decode batch {bt} d_model {dm} d_inner {di}", flush=True)
    _, state = m.prefill(td[:, :4].contiguous())
    st_sep = [(s_.clone(), c.clone()) for s_, c in state]
    lg = m.decode_step(td[:, 4].contiguous(), state)
    ssm.set_gemm_kernel(3)
    try:
        lg_sep = m.decode_step(td[:, 4].contiguous(), st_sep)
    finally:
        ssm.set_gemm_kernel(0)
    torch.cuda.synchronize()
    err = norm_err(lg.cpu().numpy(), lg_sep.cpu().numpy())
    assert err <= 1e-3, err
    for (a, b), (c, d) in zip(state, st_sep):
        assert norm_err(a.cpu().numpy(), c.cpu().numpy()) <= 1e-3
        assert torch.equal(b, d)  # the conv window holds copied inputs
    sub = tok[[0, bt - 1]]
    _, rst = oracle.lm_prefill(sub[:, :4], P, r)
    rl, _ = oracle.lm_decode_step(sub[:, 4], P, rst, r)
    err = norm_err(lg.cpu().numpy()[[0, bt - 1]], rl)
    assert err <= 1e-2, err


def test_lm_config5_full_size(dev):
    """12 layers, d_model 512, d_inner 1024, N 16, dt_rank 32, conv 4, vocab
    256, batch 16 x L 8192 prefill, then one decode step for all 16 sequences. The oracle checks
    the first 24 positions of the first and last sequences (the model is causal and the batch
    rows independent) and the decode step of those two sequences after a 24-token prefill."""
    m = ByteLM(device=dev)
    P = m.host_params()
    bt, L = 16, 8192
    rng = np.random.default_rng(0x48454C49)
    tok = rng.integers(0, 256, (bt, L)).astype(np.int32)
    td = torch.from_numpy(tok).to(dev)
    logits, state = m.prefill(td)
    torch.cuda.synchronize()
    assert torch.isfinite(logits).all()
    T = 24
    for b in (0, bt - 1):
        ref, _ = oracle.lm_prefill(tok[b:b + 1, :T], P, m.dt_rank)
        ref64, _, terms = oracle.numpy_lm_prefill(tok[b:b + 1, :T], P, m.dt_rank, return_terms=True)
        check_logits(logits[b:b + 1, :T].cpu().numpy(), ref, ref64, terms, f"prefill prefix of sequence {b}")
    lg = m.decode_step(td[:, -1], state)
    torch.cuda.synchronize()
    assert torch.isfinite(lg).all()
    sub = tok[[0, bt - 1], :T]
    _, rst = oracle.lm_prefill(sub[:, :T - 1], P, m.dt_rank)
    rl, _ = oracle.lm_decode_step(sub[:, T - 1], P, rst, m.dt_rank)
    _, rst64 = oracle.numpy_lm_prefill(sub[:, :T - 1], P, m.dt_rank)
    rl64, _, terms = oracle.numpy_lm_decode_step(sub[:, T - 1], P, rst64, m.dt_rank, return_terms=True)
    small, st2 = m.prefill(torch.from_numpy(np.ascontiguousarray(sub[:, :T - 1])).to(dev))
    g2 = m.decode_step(torch.from_numpy(np.ascontiguousarray(sub[:, T - 1])).to(dev), st2)
    torch.cuda.synchronize()
    check_logits(g2.cpu().numpy(), rl, rl64, terms, "decode after a 23-token prefill (batch 2)")


def test_decode_graph_replays_match_eager(dev):
    """The captured decode step (HIP graph) against eager decode steps from the same state, with
    eager work and synchronisation between replays; every replay is checked, bit for bit (the
    same kernels run in the same order)."""
    P = lm_params(2, 64, 128, 16, 8, 4, 256, seed=9)
    m = model_from(P, dev, dt_rank=8)
    rng = np.random.default_rng(10)
    tok = torch.from_numpy(rng.integers(0, 256, (4, 12)).astype(np.int32)).to(dev)
    _, st_eager = m.prefill(tok)
    st_graph = [(s.clone(), c.clone()) for s, c in st_eager]
    step = m.decode_graph(st_graph)
    for t in range(5):
        nxt = torch.from_numpy(rng.integers(0, 256, (4,)).astype(np.int32)).to(dev)
        want = m.decode_step(nxt, st_eager).clone()
        _ = torch.randn(1000, device=dev).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        got = step(nxt).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want), t
        for (a, b), (c, d) in zip(st_graph, st_eager):
            assert torch.equal(a, c) and torch.equal(b, d), t


def test_decode_graph_survives_workspace_growth(dev):
    """A captured decode step keeps its own workspace: a later prefill of a longer batch grows
    (replaces) the model's shared workspace and the freed block is reused by unrelated tensors;
    replays must still match eager decode steps bit for bit."""
    P = lm_params(2, 64, 128, 16, 8, 4, 256, seed=11)
    m = model_from(P, dev, dt_rank=8)
    rng = np.random.default_rng(12)
    tok = torch.from_numpy(rng.integers(0, 256, (4, 10)).astype(np.int32)).to(dev)
    _, st_eager = m.prefill(tok)
    st_graph = [(s.clone(), c.clone()) for s, c in st_eager]
    step = m.decode_graph(st_graph)
    # grow the shared workspace and scribble over whatever the allocator hands out next
    big = torch.from_numpy(rng.integers(0, 256, (8, 300)).astype(np.int32)).to(dev)
    m.prefill(big)
    junk = [torch.full((1 << 20,), 7.0, device=dev) for _ in range(8)]
    for t in range(4):
        nxt = torch.from_numpy(rng.integers(0, 256, (4,)).astype(np.int32)).to(dev)
        want = m.decode_step(nxt, st_eager).clone()
        torch.cuda.synchronize()
        got = step(nxt).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want), t
        for (a, b), (c, d) in zip(st_graph, st_eager):
            assert torch.equal(a, c) and torch.equal(b, d), t
    del junk


def test_lm_config5_decode_batch256(dev):
    """BASELINE config 5's decode leg at its own batch (256): the full 12-layer model prefills 24
    tokens per sequence, then one eager decode step and one replay of the captured step (from a
    copy of the same state). At M = 256 in_proj takes the small-M GEMM's 64-wide tiles (batch 16
    takes its 32-wide ones). The oracle checks two sequences (first and last); the eager step
    and the graph replay agree bit for bit; decode after a 23-token prefill continues it (equals
    the 24-token prefill's last position within the bf16 bar).

    Bars (check_logits): normwise 1e-2 against the same-rounding f32 oracle, or twice that
    oracle's own distance from its float64 twin where larger (through 12 layers of bf16
    intermediates a one-ulp flip anywhere propagates, and the f32 oracle itself sits that far from
    the exact value of its rounding points); componentwise against the float64 twin within a few
    bf16 ulps of each logit's term magnitudes. Decode after a 23-token prefill continues it: normwise
    2e-2 of the 24-token prefill's last position (two device evaluations that round differently)."""
    m = ByteLM(device=dev)
    P = m.host_params()
    bt, T = 256, 24
    rng = np.random.default_rng(0xC5D)
    tok = rng.integers(0, 256, (bt, T)).astype(np.int32)
    td = torch.from_numpy(tok).to(dev)
    print("case config5 decode batch 256", flush=True)
    full, _ = m.prefill(td)
    _, state = m.prefill(td[:, :T - 1].contiguous())
    st_graph = [(s.clone(), c.clone()) for s, c in state]
    lg = m.decode_step(td[:, T - 1].contiguous(), state)
    step = m.decode_graph(st_graph)
    lg_graph = step(td[:, T - 1].contiguous()).clone()
    torch.cuda.synchronize()
    assert torch.isfinite(lg).all()
    assert torch.equal(lg, lg_graph)
    for (a, b), (c, d) in zip(st_graph, state):
        assert torch.equal(a, c) and torch.equal(b, d)
    err = norm_err(lg.cpu().numpy(), full[:, T - 1].cpu().numpy())
    print(f"decode vs 24-token prefill: normwise {err:.3e}")
    assert err <= 2e-2, err
    sub = tok[[0, bt - 1]]
    _, rst = oracle.lm_prefill(sub[:, :T - 1], P, m.dt_rank)
    rl, _ = oracle.lm_decode_step(sub[:, T - 1], P, rst, m.dt_rank)
    _, rst64 = oracle.numpy_lm_prefill(sub[:, :T - 1], P, m.dt_rank)
    rl64, _, terms = oracle.numpy_lm_decode_step(sub[:, T - 1], P, rst64, m.dt_rank, return_terms=True)
    g = lg.cpu().numpy()[[0, bt - 1]]
    check_logits(g, rl, rl64, terms, "batch-256 decode, sequences 0 and 255")
