"""Integer block dots of every production engine, bit-exact, through the real entry points.

Unit-scale inputs (every weight scale 1, every activation block at d_a = 1, integer offsets; see
ksq/refcheck.py "unit-scale exactness") make each block's contribution to an output an integer,
and the inputs are sized so that the sum of all contributions' magnitudes stays below 2^24: the
fp32 output of a correct engine is then the exact integer sum in any accumulation order, so
`np.array_equal` against the exact result checks every integer block dot (and every scale,
nibble, sub-block and offset) of the engine that produced the output — not a debug kernel.
Rows alternate between dense rows (all blocks) and one-hot rows (one block; the position walks
every block of the row), so each block position is also checked on its own.  Each case asserts
the engine families the call launched (ksq_debug_last_engines), so the table below is the
evidence of which kernel serves which case.  Bars: gemm_reference.h:200-212 (Q4_0 sumi), :253-256
(Q8_0 sumi), the block formulas :175-267 and gemm_ref.py:100-153, :274-330.
"""
import os
import zlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN_LIB = os.path.join(ROOT, "tests", "dropin", "libdropin_forward.so")
TWO24 = float(2 ** 24)

# activation quant range per weight type (further limited by refcheck.unit_qmax for long rows)
QMAX_F32 = {0: 127, 1: 63, 2: 12, 3: 12, 4: 127, 5: 127, 6: 127}
QMAX_Q81 = {0: 128, 1: 63, 2: 15, 3: 15, 4: 128, 5: 128, 6: 128}


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    from ksq import _lib
    _lib.lib()
    return torch.device("cuda:0")


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _exact(wtype, a_blocks, w, q8s=False):
    from ksq import refcheck
    ref, bound = refcheck.exact_gemm(wtype, a_blocks, w, q8s)
    assert bound.max() < TWO24, f"test inputs too large for exact fp32 sums: {bound.max():.3e}"
    return ref.astype(np.float32)


def _inputs(wtype, g, M, N, K, atype, onehot, q6k_scale=32):
    """(weights, activation input, the block_q8_1 / block_q8s blocks the engine must see)."""
    from ksq import refcheck
    from oracle import oracle
    w = refcheck.unit_weights(wtype, g, N, K, q6k_scale=q6k_scale)
    qmax = min(QMAX_F32[wtype], refcheck.unit_qmax(wtype, K))
    if atype in (0, 2):            # fp32, quantised by the library (block_q8_1 / block_q8s rules)
        x = refcheck.unit_activations(g, M, K, qmax=qmax, onehot=onehot)
        blocks = oracle.quantize_q8s(x) if atype == 2 else oracle.quantize_q8_1(x)
        return w, x, blocks
    if atype == 3:
        a = refcheck.unit_q8s(g, M, K, qmax=min(QMAX_Q81[wtype], 127, qmax), onehot=onehot)
        return w, a, a
    if atype == 4:                 # fp16: the fused FP16 kernels' quantiser gives d = 1, q = x
        x = refcheck.unit_activations(g, M, K, qmax=qmax, onehot=onehot).astype(np.float16)
        return w, x, oracle.quantize_q8_1_variant(x, 3)
    smax = 512 if wtype in (2, 3) or K > 8192 else 2048
    a = refcheck.unit_q8_1(g, M, K, qmax=min(QMAX_Q81[wtype], qmax if qmax < 127 else 128), onehot=onehot, smax=smax)
    return w, a, a


def _gemm(dev, wtype, atype, w, x, M, N, K, path=0, cfg=0):
    import torch
    from ksq import _lib, ops
    L = _lib.lib()
    assert L.ksq_set_path(path) == 0 and L.ksq_set_mmq_config(cfg) == 0
    try:
        y = ops.gemm(wtype, atype, _t(w, dev), _t(x, dev), M, N, K)
        eng = ops.last_engines()
        torch.cuda.synchronize()
    finally:
        L.ksq_set_path(0)
        L.ksq_set_mmq_config(0)
    return y.cpu().numpy(), eng


def _void(dev, entry, w, x, M, N, K):
    """A drop-in symbol called as the reference harness calls its kernel: device pointers, no
    stream (the null stream), no workspace; then synchronise and read the status."""
    import torch
    from ksq import _lib, ops
    L = _lib.lib()
    wt, xt = _t(w, dev), _t(x, dev)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    getattr(L, entry)(wt.data_ptr(), xt.data_ptr(), y.data_ptr(), M, N, K)
    eng = ops.last_engines()
    torch.cuda.synchronize()
    assert L.ksq_last_error() == 0, L.ksq_last_error_message().decode()
    return y.cpu().numpy(), eng


def _spot_oracle(oracle, wtype, blocks, w, y, rows, K):
    """The C oracle's fp64 block formula on a few rows: exact for these integer inputs."""
    ref = oracle.gemm_f64(wtype, blocks[rows], w, len(rows), w.shape[0], K)
    assert np.array_equal(y[rows], ref.astype(np.float32))


# ------------------------------------------------------------------ BASELINE configs, drop-in entries
F32_ENTRY = {0: "gemm_w4a32c8_q4_0_fp32_int8", 1: "gemm_w8a32c8_q8_0_fp32_int8", 2: "gemm_w4a32c8_q4_k_fp32_int8",
             3: "gemm_w6a32c8_q6_k_fp32_int8", 4: "gemm_w4a32c8_q4_1_fp32_int8", 5: "gemm_w5a32c8_q5_0_fp32_int8",
             6: "gemm_w5a32c8_q5_1_fp32_int8"}
Q81_ENTRY = {0: "ksq_gemm_q4_0_q8_1", 1: "ksq_gemm_q8_0_q8_1", 2: "ksq_gemm_q4_k_q8_1", 3: "ksq_gemm_q6_k_q8_1",
             4: "ksq_gemm_q4_1_q8_1", 5: "ksq_gemm_q5_0_q8_1", 6: "ksq_gemm_q5_1_q8_1"}

CONFIG_CASES = [
    # name, wtype, M, N, K, activation input, engines the call must launch
    ("c0_q4_0_m1_f32", 0, 1, 4096, 4096, "f32", {"gemv_direct_fq"}),
    ("c0_q4_0_m1_q81", 0, 1, 4096, 4096, "q81", {"gemv_direct"}),
    ("c1_q8_0_m1_f32", 1, 1, 4096, 4096, "f32", {"gemv_direct_fq"}),
    ("c1_q8_0_m1_q81", 1, 1, 4096, 4096, "q81", {"gemv_direct"}),
    ("c1_q8_0_m8_f32", 1, 8, 4096, 4096, "f32", {"quantize", "skinny"}),
    ("c1_q8_0_m8_q81", 1, 8, 4096, 4096, "q81", {"skinny"}),
    ("c1_q8_0_m32_f32", 1, 32, 4096, 4096, "f32", {"quantize", "skinny"}),
    ("c1_q8_0_m32_q81", 1, 32, 4096, 4096, "q81", {"skinny"}),
    ("c2_q4_0_m2048_f32", 0, 2048, 4096, 4096, "f32", {"quantize", "mmq_planar"}),
    ("c2_q4_0_m2048_q81", 0, 2048, 4096, 4096, "q81", {"mmq1"}),
    ("c3_q4_k_m128_f32", 2, 128, 14336, 4096, "f32", {"quantize", "mmq7", "splitk"}),
    ("c3_q4_k_m128_q81", 2, 128, 14336, 4096, "q81", {"mmq7", "splitk"}),
    ("c3_q6_k_m128_f32", 3, 128, 14336, 4096, "f32", {"quantize", "mmq3"}),
    ("c3_q6_k_m128_q81", 3, 128, 14336, 4096, "q81", {"mmq3"}),
]


@pytest.mark.parametrize("name,wtype,M,N,K,inp,engines", CONFIG_CASES, ids=[c[0] for c in CONFIG_CASES])
def test_exact_baseline_configs(dev, oracle, name, wtype, M, N, K, inp, engines):
    """BASELINE configs 0-3 at full size through the drop-in void symbols: every output equals
    the exact integer result; M = 1 runs one dense call and one-hot calls at block positions
    0, 1, the middle, the last two and a random one."""
    from ksq import refcheck
    g = np.random.default_rng(zlib.crc32(name.encode()))
    atype = 0 if inp == "f32" else 1
    entry = F32_ENTRY[wtype] if inp == "f32" else Q81_ENTRY[wtype]
    nb = K // 32
    if M == 1:
        patterns = [None] + [np.array([b]) for b in (0, 1, nb // 2, nb - 2, nb - 1, int(g.integers(0, nb)))]
    else:
        patterns = [refcheck.onehot_pattern(M, nb, every=2, seed=int(g.integers(0, nb)))]
    w = None
    for oh in patterns:
        w_new, x, blocks = _inputs(wtype, g, M, N, K, atype, oh)
        w = w_new if w is None else w          # one weight matrix per case
        y, eng = _void(dev, entry, w, x, M, N, K)
        assert eng == engines, (name, eng)
        assert np.array_equal(y, _exact(wtype, blocks, w)), (name, None if oh is None else oh[:4])
    _spot_oracle(oracle, wtype, blocks, w, y, np.array([0, M - 1]) if M > 1 else np.array([0]), K)


def test_exact_moe_config4(dev, oracle):
    """Config 4 (512 tokens, 8 experts of Q4_0 14336 x 4096, top-2) through the grouped GEMM with
    caller routing: routing weights 1 and 0.5 keep every output an exact integer multiple of 1/2;
    dense and one-hot token rows; each expert's rows checked against the exact products."""
    import torch
    from ksq import ops, refcheck
    T, E, N, K, top_k = 512, 8, 14336, 4096, 2
    g = np.random.default_rng(4400)
    nb = K // 32
    w = np.stack([refcheck.unit_weights(0, g, N, K) for _ in range(E)])
    x = refcheck.unit_activations(g, T, K, qmax=127, onehot=refcheck.onehot_pattern(T, nb, every=2, seed=5))
    ids = np.stack([g.choice(E, size=top_k, replace=False) for _ in range(T)]).astype(np.int32)
    wts = np.tile(np.array([1.0, 0.5], np.float32), (T, 1))
    y = ops.moe_gemm_routed(0, _t(w, dev), _t(x, dev), _t(ids, dev), _t(wts, dev), T, N, K, E)
    eng = ops.last_engines()
    torch.cuda.synchronize()
    # ~128 rows per expert: the LDS-DMA kernel's 128-row tiles over expert-sorted planar rows
    assert eng == {"quantize", "moe_group", "moe_planar"}, eng
    a = oracle.quantize_q8_1(x)
    ref = np.zeros((T, N))
    for e in range(E):
        tok, slot = np.nonzero(ids == e)
        if len(tok) == 0:
            continue
        ye, bound = refcheck.exact_gemm(0, a[tok], w[e])
        assert bound.max() < TWO24
        ref[tok] += wts[tok, slot][:, None] * ye
    assert np.array_equal(y.cpu().numpy(), ref.astype(np.float32))


# ------------------------------------------------------------------ every engine, forced
ALL = [0, 1, 2, 3, 4, 5, 6]
LEGACY = [0, 1, 4, 5, 6]


def _engine_cases():
    """(id, wtype, M, N, K, atype, path, cfg, expected engines, weight byte offset)."""
    cases = []
    for wt in ALL:
        kq = wt in (2, 3)
        # decode, pre-quantised (path 1)
        cases.append((f"dec_m1_w{wt}", wt, 1, 256, 2048, 1, 1, 0, {"gemv_kq" if kq else "gemv_direct"}, 0))
        cases.append((f"dec_m2_w{wt}", wt, 2, 256, 2048, 1, 1, 0,
                      {"gemv_row" if wt == 3 else "gemv_kq" if kq else "gemv_direct"}, 0))
        cases.append((f"dec_m5_w{wt}", wt, 5, 2048, 2048, 1, 1, 0, {"gemv_row" if wt == 3 else "gemv_mr"}, 0))
        cases.append((f"dec_m3_smallN_w{wt}", wt, 3, 200, 1024, 1, 1, 0, {"gemv_row" if wt == 3 else "gemv_mr"}, 0))
        cases.append((f"dec_m8_w{wt}", wt, 8, 2048, 1024, 1, 1, 0, {"gemv_row" if wt == 3 else "gemv_mr"}, 0))
        # decode, fp32 input (fused quantisation where it applies)
        cases.append((f"decf_m1_w{wt}", wt, 1, 256, 1024, 0, 1, 0, {"gemv_row_fq" if kq else "gemv_direct_fq"}, 0))
        cases.append((f"decf_m4_w{wt}", wt, 4, 512, 1024, 0, 1, 0,
                      {"quantize", "gemv_row" if wt == 3 else "gemv_mr"} if kq else {"gemv_mr_fq"}, 0))
        # MFMA GEMM, every tile configuration (K-quants take the automatic tile for 4 and 6)
        # (the K-step-4 tiles split this 4-workgroup grid in two along K)
        # (automatic for M = 150-200: Q4_K the 64 x 128 tile, Q6_K 64 x 64)
        auto = "mmq7" if wt == 2 else "mmq3"
        for cfg in range(1, 8):
            eng = {f"mmq{cfg}", "splitk"} if cfg in (4, 6) else {f"mmq{cfg}"}
            cases.append((f"mmq_cfg{cfg}_w{wt}", wt, 150, 136, 512, 1, 2, cfg, {auto} if kq and cfg in (4, 6) else eng,
                          0))
        cases.append((f"mmqf_w{wt}", wt, 200, 384, 1024, 0, 2, 0, {"quantize", auto if kq else "mmq3", "splitk"}, 0))
    for wt in LEGACY:
        cases.append((f"dec_oddnb_w{wt}", wt, 1, 200, 1056, 1, 1, 0, {"gemv_row"}, 0))
        cases.append((f"dec_long_w{wt}", wt, 1, 64, 20480, 1, 1, 0, {"gemv_row"}, 0))
        cases.append((f"dec_unaligned_w{wt}", wt, 1, 100, 1024, 1, 1, 0, {"gemv_row"}, 2))
        cases.append((f"decf_oddnb_w{wt}", wt, 1, 100, 1056, 0, 1, 0, {"gemv_row_fq"}, 0))
        for M in (1, 3, 8):
            cases.append((f"skinny_m{M}_w{wt}", wt, M, 200, 1024, 1, 3, 0, {"skinny"}, 0))
        # 9-32 rows (the 16x16x32-MFMA form over the shared activation pieces), ragged rows
        for M in (12, 17, 32):
            cases.append((f"skinny_m{M}_w{wt}", wt, M, 200, 1152, 1, 3, 0, {"skinny"}, 0))
        # weights 4-byte aligned only: Q8_0 off its row-chunk staging onto the per-lane windows
        cases.append((f"skinny_m20_woff4_w{wt}", wt, 20, 130, 1024, 1, 3, 0, {"skinny"}, 4))
        # one K step in all (fewer steps than waves: the idle waves add zeros), N below one workgroup
        cases.append((f"skinny_m20_k128_w{wt}", wt, 20, 12, 128, 1, 3, 0, {"skinny"}, 0))
    # the LDS-DMA GEMM (fp32 activations quantised to planar block_q8_1; Q4_0 / Q4_1): split in
    # two along K, with an even (4) and an odd (5) number of 4-block steps per split; ragged M, N
    for wt in (0, 4):
        for K in (1024, 1280):
            cases.append((f"mmqp_k{K}_w{wt}", wt, 200, 330, K, 0, 2, 8, {"quantize", "mmq_planar", "splitk"}, 0))
        # a single row and a ragged 33 rows in one 128-row tile (rows past M read row M-1)
        for M in (1, 33):
            cases.append((f"mmqp_m{M}_w{wt}", wt, M, 136, 512, 0, 2, 8, {"quantize", "mmq_planar"}, 0))
    cases.append(("splitk_w0", 0, 32, 1024, 8192, 1, 2, 0, {"mmq5", "splitk"}, 0))
    cases.append(("splitk_w1", 1, 32, 1024, 8192, 1, 2, 0, {"mmq3", "splitk"}, 0))
    # the native W8A8C8 operator's block_q8s activations: fp32 (its quantiser) and pre-quantised
    for M, path, eng in ((1, 1, {"gemv_direct_fq"}), (5, 3, {"quantize", "skinny"}),
                         (150, 2, {"quantize", "mmq3", "splitk"})):
        cases.append((f"q8s_f32_m{M}", 1, M, 256, 1024, 2, path, 0, eng, 0))
    for M, path, eng in ((2, 1, {"gemv_direct"}), (6, 3, {"skinny"}), (150, 2, {"mmq3", "splitk"})):
        cases.append((f"q8s_m{M}", 1, M, 256, 1024, 3, path, 0, eng, 0))
    # fp16 activations (quantised by the fused FP16 kernels' rules)
    # (1-2 rows: quantised inside the decode kernel's workgroups, into LDS)
    for M, path, eng in ((1, 1, {"gemv_direct_fq"}), (2, 0, {"gemv_direct_fq"}), (4, 3, {"quantize", "skinny"}),
                         (150, 2, {"quantize", "mmq3", "splitk"})):
        cases.append((f"f16_m{M}", 0, M, 256, 1024, 4, path, 0, eng, 0))
    for M in (1, 2):
        cases.append((f"f16_row_m{M}", 4, M, 256, 1024, 4, 1, 0, {"gemv_row_fq"}, 2))
    # 3-8 fp16 rows: quantised inside the multi-row decode kernel's workgroups (no quantise launch)
    for wt in LEGACY:
        for M in (3, 8):
            cases.append((f"f16_mr_m{M}_w{wt}", wt, M, 256, 1024, 4, 0, 0, {"gemv_mr_fq"}, 0))
    return cases


ENGINE_CASES = _engine_cases()


@pytest.mark.parametrize("cid,wtype,M,N,K,atype,path,cfg,engines,woff", ENGINE_CASES,
                         ids=[c[0] for c in ENGINE_CASES])
def test_exact_engine(dev, oracle, cid, wtype, M, N, K, atype, path, cfg, engines, woff):
    """One engine (decode kernels, small-batch MFMA, every MFMA tile, split-K) per case, forced
    with the routing knobs: outputs equal the exact integer result, dense and one-hot rows."""
    from ksq import refcheck
    g = np.random.default_rng(zlib.crc32(cid.encode()))
    nb = K // 32
    oh = refcheck.onehot_pattern(M, nb, every=2, seed=3) if M > 1 else None
    w, x, blocks = _inputs(wtype, g, M, N, K, atype, oh)
    want = _exact(wtype, blocks, w, q8s=atype in (2, 3))
    if woff:
        # the same weights at a 2-byte offset: the generic (unaligned) decode path
        buf = np.zeros(w.size + woff, np.uint8)
        buf[woff:] = w.reshape(-1)
        import torch
        from ksq import _lib, ops
        L = _lib.lib()
        bt = _t(buf, dev)
        xt = _t(x, dev)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        assert L.ksq_set_path(path) == 0
        try:
            from ksq._lib import check
            check(L.ksq_gemm(wtype, atype, bt.data_ptr() + woff, xt.data_ptr(), y.data_ptr(), M, N, K, None, 0,
                             torch.cuda.current_stream().cuda_stream))
            eng = ops.last_engines()
            torch.cuda.synchronize()
        finally:
            L.ksq_set_path(0)
        y = y.cpu().numpy()
    else:
        y, eng = _gemm(dev, wtype, atype, w, x, M, N, K, path=path, cfg=cfg)
    assert eng == engines, (cid, eng)
    assert np.array_equal(y, want), cid


def test_engine_table_covers_every_engine():
    """The forced cases above (plus the MoE and fused FP16 cases below, and the dequantise-then-fp32
    GEMM of tests/test_gpu_w16.py) reach every kernel family the library has."""
    from ksq import _lib
    seen = set().union(*(c[8] for c in ENGINE_CASES)) | {"moe_tile64", "moe_tile128", "moe_planar", "moe_combine",
                                                          "moe_route", "moe_group", "transpose", "w16"}
    assert seen == set(_lib.ENG), set(_lib.ENG) - seen


# ------------------------------------------------------------------ MoE engines
@pytest.mark.parametrize("wtype", LEGACY)
@pytest.mark.parametrize("T,E,top_k,tile,skew", [(96, 4, 2, 64, False), (96, 4, 3, 64, False),
                                                 (800, 4, 2, 64, False), (300, 4, 2, 64, True),
                                                 (260, 4, 3, 64, True)])
def test_exact_moe_engines(dev, wtype, T, E, top_k, tile, skew):
    """Grouped GEMM per block type, and the top_k > 2 combine; with top_k = 3 one slot of one
    token carries an out-of-range expert id, which contributes nothing.  From 96 entries per
    expert on, Q4_0 / Q4_1 run the LDS-DMA kernel on 128-row tiles of expert-sorted planar rows;
    skewed routing (expert shares 0.55 / 0.3 / 0.1 / 0.05) leaves tiles with 1-4 of their 32-row
    sub-tiles holding rows, and experts whose rows end mid-tile.  The other types (and fewer
    rows) take mmq_kernel's 64-row tiles."""
    import torch
    from ksq import ops, refcheck
    from oracle import oracle
    if tile == 128 and wtype not in (0, 4):
        pytest.skip("128-row grouped tiles are used for the nibble types only")
    N, K = 256, 512
    g = np.random.default_rng(4500 + 10 * wtype + top_k)
    w = np.stack([refcheck.unit_weights(wtype, g, N, K) for _ in range(E)])
    x = refcheck.unit_activations(g, T, K, qmax=QMAX_F32[wtype], onehot=refcheck.onehot_pattern(T, K // 32))
    p = np.array([0.55, 0.3, 0.1, 0.05]) if skew else None
    ids = np.stack([g.choice(E, size=top_k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    if top_k == 3:
        ids[7, 1] = E
    wts = (2.0 ** -g.integers(0, 3, size=(T, top_k))).astype(np.float32)
    y = ops.moe_gemm_routed(wtype, _t(w, dev), _t(x, dev), _t(ids, dev), _t(wts, dev), T, N, K, E)
    eng = ops.last_engines()
    torch.cuda.synchronize()
    grouped = "moe_planar" if wtype in (0, 4) and T * top_k >= 96 * E else f"moe_tile{tile}"
    want_eng = {"quantize", "moe_group", grouped} | ({"moe_combine"} if top_k > 2 else set())
    assert eng == want_eng, eng
    a = oracle.quantize_q8_1(x)
    ref = np.zeros((T, N))
    for e in range(E):
        tok, slot = np.nonzero(ids == e)
        if len(tok):
            ye, bound = refcheck.exact_gemm(wtype, a[tok], w[e])
            assert bound.max() < TWO24
            ref[tok] += wts[tok, slot][:, None] * ye
    assert np.array_equal(y.cpu().numpy(), ref.astype(np.float32))


# ------------------------------------------------------------------ the other drop-in symbols
DROPIN_CASES = [(e, wt, "f32") for wt, e in F32_ENTRY.items()] + [(e, wt, "q81") for wt, e in Q81_ENTRY.items()] + \
    [("gemm_w8a8c8_q8_0_q8_1", 1, "q8s")]


@pytest.mark.parametrize("entry,wtype,inp", DROPIN_CASES, ids=[c[0] for c in DROPIN_CASES])
@pytest.mark.parametrize("M", [1, 5, 64])
def test_exact_dropin_symbols(dev, entry, wtype, inp, M):
    """Every void symbol of the reference signature, called with device pointers on the null
    stream with the library's own pool (M = 1 decode, 5 small batch, 64 MFMA)."""
    from ksq import refcheck
    N, K = 512, 2048
    g = np.random.default_rng(4600 + M + 7 * wtype)
    atype = {"f32": 0, "q81": 1, "q8s": 2}[inp]
    w, x, blocks = _inputs(wtype, g, M, N, K, atype, refcheck.onehot_pattern(M, K // 32) if M > 1 else None)
    y, _ = _void(dev, entry, w, x, M, N, K)
    assert np.array_equal(y, _exact(wtype, blocks, w, q8s=inp == "q8s")), entry


def test_moe_void_entry_matches_routing_entry(dev, oracle):
    """moe_w4a32c8_q4_0_fp32_int8 (null stream, library pool) gives bit for bit what ksq_moe_gemm
    gives for the same routing (top-2 outputs get exactly two additions onto zero, so no order
    dependence), and the routing matches the oracle's softmax / top-k."""
    import torch
    from ksq import _lib, ops, synth
    T, E, N, K, top_k = 200, 8, 512, 1024, 2
    g = np.random.default_rng(4700)
    w = np.concatenate([synth.weights(0, g, N, K) for _ in range(E)])
    x = synth.activations(g, T, K)
    lg = synth.router_logits(g, T, E)
    wt, xt, lt = _t(w, dev), _t(x, dev), _t(lg, dev)
    y1, ids, wts = ops.moe_gemm(0, wt, xt, lt, T, N, K, E, top_k, return_routing=True)
    y2 = torch.full((T, N), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    _lib.lib().moe_w4a32c8_q4_0_fp32_int8(wt.data_ptr(), xt.data_ptr(), lt.data_ptr(), y2.data_ptr(), T, N, K, E,
                                          top_k)
    torch.cuda.synchronize()
    assert _lib.lib().ksq_last_error() == 0
    assert torch.equal(y1, y2)
    rid, rw = oracle.moe_route(lg, top_k)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.allclose(wts.cpu().numpy(), rw, rtol=1e-6, atol=0)


def test_fp16_fused_orientation_exact(dev):
    """ksq_gemm_q4_0_fp16_fused (M weight rows, fp16 activations [N][K], output [M][N]) with a
    caller workspace and with the pool: the transposed exact result."""
    import torch
    from ksq import ops, refcheck
    g = np.random.default_rng(4800)
    Mw, Na, K = 384, 40, 1024
    w, xh, blocks = _inputs(0, g, Na, Mw, K, 4, refcheck.onehot_pattern(Na, K // 32))
    want = _exact(0, blocks, w).T
    ws = torch.empty(ops.gemm_q4_0_fp16_fused_workspace_size(Mw, Na, K) + 256, dtype=torch.uint8, device=dev)
    off = (-ws.data_ptr()) % 256
    y1 = ops.gemm_q4_0_fp16_fused(_t(w, dev), _t(xh, dev), Mw, Na, K, workspace=ws[off:])
    assert "transpose" in ops.last_engines()
    y2 = ops.gemm_q4_0_fp16_fused(_t(w, dev), _t(xh, dev), Mw, Na, K)
    torch.cuda.synchronize()
    assert np.array_equal(y1.cpu().numpy(), want)
    assert np.array_equal(y2.cpu().numpy(), want)


@pytest.mark.parametrize("Mw,Na,K,engines", [
    (512, 1, 1024, {"gemv_direct_fq"}),          # decode: fp16 quantised in LDS, [M][N] stored directly
    (4096, 2, 2048, {"gemv_direct_fq"}),
    # 3-8 activation rows: fp16 quantised in LDS by the multi-row decode kernel, [M][N] stored
    # directly (the reference tiles 4 activation columns per block: gemm_fused.cuh:157-162)
    (768, 3, 4096, {"gemv_mr_fq"}),
    (1024, 4, 2048, {"gemv_mr_fq"}),
    (1024, 8, 1024, {"gemv_mr_fq"}),
    # past the in-workgroup quantisation's work limit: one quantise launch, then the multi-row
    # decode kernel storing [M][N] directly (no transpose; ksq_gemm itself would take the
    # small-batch MFMA kernel at 8 rows and the split MFMA GEMM at 14336 x 4096 x 8)
    (4096, 5, 4096, {"quantize", "gemv_mr"}),
    (14336, 3, 4096, {"quantize", "gemv_mr"}),
    (4096, 8, 4096, {"quantize", "gemv_mr"}),
    (14336, 8, 4096, {"quantize", "gemv_mr"}),
    (4096, 512, 1024, {"quantize", "mmq3"}),     # MFMA GEMM writing its tiles transposed
    (384, 40, 1024, {"quantize", "mmq3", "splitk", "transpose"}),   # split-K: [N][M], then transposed
])
def test_fp16_fused_routes_exact(dev, Mw, Na, K, engines):
    """Each route of ksq_gemm_q4_0_fp16_fused gives the exact transposed result and launches the
    kernels named (no workspace and no transpose for decode shapes and for the unsplit GEMM)."""
    import torch
    from ksq import ops, refcheck
    g = np.random.default_rng(4900 + Na)
    w, xh, blocks = _inputs(0, g, Na, Mw, K, 4, refcheck.onehot_pattern(Na, K // 32))
    want = _exact(0, blocks, w).T
    y = ops.gemm_q4_0_fp16_fused(_t(w, dev), _t(xh, dev), Mw, Na, K)
    eng = ops.last_engines()
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), want)
    assert eng == engines, eng


def test_dropin_forwarding_module(dev):
    """The forwarding kernel.cpp a maintainer compiles in place of a definition's kernel.cu
    (tests/dropin/kernel.cpp, built by __graft_entry__.build() with hipcc against include/ksq.h
    and linked with -lksq) resolves the definition's entry points in libksq and runs them."""
    import ctypes

    import torch
    from ksq import refcheck
    assert os.path.exists(DROPIN_LIB), "tests/dropin/libdropin_forward.so is built by __graft_entry__.build()"
    D = ctypes.CDLL(DROPIN_LIB)
    D.dropin_forward.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_int]
    D.dropin_forward.restype = ctypes.c_int
    g = np.random.default_rng(4900)
    for entry, wtype, atype in (("gemm_w4a32c8_q4_0_fp32_int8", 0, 0), ("gemm_w8a32c8_q8_0_fp32_int8", 1, 0),
                                ("gemm_w4a32c8_q4_1_fp32_int8", 4, 0), ("gemm_w8a8c8_q8_0_q8_1", 1, 2)):
        M, N, K = 7, 1024, 4096
        w, x, blocks = _inputs(wtype, g, M, N, K, atype, refcheck.onehot_pattern(M, K // 32))
        wt, xt = _t(w, dev), _t(x, dev)
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        st = D.dropin_forward(entry.encode(), wt.data_ptr(), xt.data_ptr(), y.data_ptr(), M, N, K)
        torch.cuda.synchronize()
        assert st == 0, entry
        assert np.array_equal(y.cpu().numpy(), _exact(wtype, blocks, w, q8s=atype == 2)), entry
    assert D.dropin_forward(b"no_such_entry", None, None, None, 1, 1, 32) == -1
