"""Kernel-level parity through the C ABI (device buffers from torch, plain pointers in)."""
import ctypes as C

import numpy as np
import pytest
import torch

import malaga_amd as M
import oracle as O
from malaga_amd import _lib

pytestmark = pytest.mark.gpu
F32, F16, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 8, 12, 13, 14


@pytest.fixture(scope="module")
def ctx():
    return M._Ctx(0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def ptr(t):
    return C.c_void_p(t.data_ptr())


def upload(ctx, t, blocks, N, K):
    h = C.c_void_p()
    _lib.check(ctx.lib.mlg_matrix_upload(ctx.h, t, N, K, blocks.ctypes.data, C.byref(h)))
    return h


def bound(x, w):
    """|y| error scale: sum_k |x_k| |w_nk| (float64)."""
    return np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T


# BASELINE config 2 shapes at 600M: fused QKV 3072 x 1024, FFN-up 4096 x 1024, FFN-down 1024 x 4096
CASES = [(t, N, K) for t in (Q4_K, Q5_K, Q6_K, Q8_0) for (N, K) in ((3072, 1024), (4096, 1024), (1024, 4096),
                                                                  (517, 256))] + \
        [(F16, 192, 64), (F32, 192, 64), (F16, 130, 128), (F32, 128, 128)]


@pytest.mark.parametrize("t,N,K", CASES)
def test_gemv_matches_dequantized_dot(ctx, t, N, K):
    rng = np.random.default_rng(N + K + t)
    wf = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    blocks = M.quantize(t, wf)
    w = upload(ctx, t, blocks, N, K)
    try:
        wd = O.dequant(t, blocks, N * K).reshape(N, K)
        maxb = ctx.lib.mlg_gemv_max_batch(w)
        assert maxb >= 1
        for b in sorted({1, maxb}):
            x = rng.normal(0, 1, (b, K)).astype(np.float32)
            bias = rng.normal(0, 0.1, N).astype(np.float32)
            xd, yd, bd = dev(x), torch.zeros((b, N), device="cuda"), dev(bias)
            _lib.check(ctx.lib.mlg_gemv(w, ptr(xd), b, ptr(yd), ptr(bd), 0, None))
            torch.cuda.synchronize()
            ref = O.gemv(t, blocks, N, K, x) + bias
            err = np.abs(yd.cpu().numpy() - ref)
            assert (err <= 2e-6 * bound(x, wd) + 1e-6).all(), (b, err.max())
            # relu epilogue
            _lib.check(ctx.lib.mlg_gemv(w, ptr(xd), b, ptr(yd), ptr(bd), 1, None))
            torch.cuda.synchronize()
            assert (yd.cpu().numpy() >= 0).all()
    finally:
        ctx.lib.mlg_matrix_free(w)


@pytest.mark.parametrize("t,N,K", [(Q4_K, 1000, 1024), (Q6_K, 300, 512), (Q8_0, 256, 1024), (F32, 96, 64)])
def test_gemm_matches_dequantized_dot(ctx, t, N, K):
    rng = np.random.default_rng(7 + t)
    wf = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    blocks = M.quantize(t, wf)
    w = upload(ctx, t, blocks, N, K)
    try:
        wd = O.dequant(t, blocks, N * K).reshape(N, K)
        for M_ in (1, 37, 70):
            x = rng.normal(0, 1, (M_, K)).astype(np.float32)
            xd, yd = dev(x), torch.zeros((M_, N), device="cuda")
            _lib.check(ctx.lib.mlg_gemm(w, ptr(xd), M_, ptr(yd), None, 0, None))
            torch.cuda.synchronize()
            ref = O.gemv(t, blocks, N, K, x)
            assert (np.abs(yd.cpu().numpy() - ref) <= 2e-6 * bound(x, wd) + 1e-6).all()
    finally:
        ctx.lib.mlg_matrix_free(w)


@pytest.mark.parametrize("t,N,K", [(Q4_K, 200, 1024), (Q5_K, 130, 512), (Q6_K, 70, 2048), (Q8_0, 64, 768),
                                   (F16, 90, 256), (Q4_K, 16400, 512)])
def test_gemm_mfma_tiles_bias_relu_residual(ctx, t, N, K):
    """The MFMA GEMM (K % 256 == 0) over every X-tile size (16 / 32 / 64 rows), partial
    tiles in M and N, with bias, ReLU and an in-place residual (R = Y); small grids
    split K over workgroups (fixed-order reduction), N = 16400 runs unsplit."""
    rng = np.random.default_rng(31 + t)
    wf = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    blocks = M.quantize(t, wf)
    w = upload(ctx, t, blocks, N, K)
    try:
        wd = O.dequant(t, blocks, N * K).reshape(N, K)
        bias = rng.normal(0, 0.1, N).astype(np.float32)
        bd = dev(bias)
        for M_ in (3, 16, 29, 32, 64, 100):
            x = (rng.normal(0, 1, (M_, K)) * rng.uniform(0.01, 30, (M_, 1))).astype(np.float32)
            r0 = rng.normal(0, 1, (M_, N)).astype(np.float32)
            xd, yd = dev(x), dev(r0)
            for relu in (0, 1):
                yd.copy_(torch.from_numpy(r0))
                _lib.check(ctx.lib.mlg_gemm_resid(w, ptr(xd), M_, ptr(yd), ptr(bd), relu, ptr(yd), None))
                torch.cuda.synchronize()
                ref = O.gemv(t, blocks, N, K, x) + bias + r0
                if relu:
                    ref = np.maximum(ref, 0)
                tol = 2e-6 * (bound(x, wd) + np.abs(bias) + np.abs(r0)) + 1e-6
                assert (np.abs(yd.cpu().numpy() - ref) <= tol).all(), (M_, relu)
    finally:
        ctx.lib.mlg_matrix_free(w)


@pytest.mark.parametrize("t,N,K", [(Q4_K, 12300, 512), (Q5_K, 12300, 256), (Q6_K, 6150, 512), (Q8_0, 6144, 256),
                                   (F16, 12290, 256)])
def test_gemm_wide_tiles(ctx, t, N, K):
    """M > 32 with many W rows runs the wide-tile kernel (8 waves x 32 rows of W per
    workgroup) once ceil(N / 256) * ceil(M / 64) >= 96: partial tiles in M and N,
    bias, ReLU, residual; q4_K at M = 200 also splits K (gemm + reduction)."""
    rng = np.random.default_rng(43 + t)
    wf = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    blocks = M.quantize(t, wf)
    w = upload(ctx, t, blocks, N, K)
    try:
        wd = O.dequant(t, blocks, N * K).reshape(N, K)
        bias = rng.normal(0, 0.1, N).astype(np.float32)
        bd = dev(bias)
        for M_ in (200, 2100 if N < 8000 else 1100):
            x = (rng.normal(0, 1, (M_, K)) * rng.uniform(0.01, 30, (M_, 1))).astype(np.float32)
            r0 = rng.normal(0, 1, (M_, N)).astype(np.float32)
            xd, yd = dev(x), dev(r0)
            _lib.check(ctx.lib.mlg_gemm_resid(w, ptr(xd), M_, ptr(yd), ptr(bd), 1, ptr(yd), None))
            torch.cuda.synchronize()
            ref = np.maximum(O.gemv(t, blocks, N, K, x) + bias + r0, 0)
            tol = 2e-6 * (bound(x, wd) + np.abs(bias) + np.abs(r0)) + 1e-6
            assert (np.abs(yd.cpu().numpy() - ref) <= tol).all(), M_
    finally:
        ctx.lib.mlg_matrix_free(w)


@pytest.mark.parametrize("t,K", [(Q6_K, 1024), (Q4_K, 1024), (Q8_0, 512), (Q5_K, 2048), (Q6_K, 2048)])
def test_gemm_argmax_batched_lm_head(ctx, t, K):
    """Batched LM head (5..64 rows): per-workgroup argmax partials merged on the host equal
    the argmax of the oracle's logits; ties -> lowest index; mask_id is skipped.  Up to 32
    rows X is resident in LDS (17..32 rows need K <= 1024, else the form is refused: 0
    partials); 33..64 rows run the wide-tile GEMM with the argmax epilogue, any K."""
    rng = np.random.default_rng(5 + t)
    N = 20000
    wf = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    # tied dominant rows: 4300 / 4321 / 4325 share a 256-row workgroup of the wide-tile
    # kernel (two waves; 4321 and 4325 one wave's lanes), 15000 is in another
    wf[4300] = wf[4321] = wf[4325] = wf[15000] = rng.normal(0, 0.5, K).astype(np.float32)
    blocks = M.quantize(t, wf)
    w = upload(ctx, t, blocks, N, K)
    try:
        for M_ in (5, 16, 17, 32, 33, 64):
            parts = ctx.lib.mlg_gemm_argmax_parts(w, M_)
            if K > 1024 and 16 < M_ <= 32:
                assert parts == 0
                continue
            assert parts > 0
            x = rng.normal(0, 1, (M_, K)).astype(np.float32)
            x[0] = np.abs(x[0]) * np.sign(wf[4321])
            ref = O.gemv(t, blocks, N, K, x)
            for mask in (-1, 4300):
                pv = torch.zeros((M_, parts), device="cuda")
                pi = torch.zeros((M_, parts), dtype=torch.int32, device="cuda")
                _lib.check(ctx.lib.mlg_gemm_argmax(w, ptr(dev(x)), M_, mask, ptr(pv), ptr(pi), None))
                torch.cuda.synchronize()
                v, i = pv.cpu().numpy(), pi.cpu().numpy().view(np.uint32)
                r = ref.copy()
                if mask >= 0:
                    r[:, mask] = -np.inf
                for m in range(M_):
                    best = v[m].max()
                    got = int(i[m][v[m] == best].min())
                    want = int(np.argmax(r[m]))
                    # near-ties within f32 rounding may legitimately resolve either way
                    assert got == want or abs(r[m][got] - r[m][want]) <= 2e-6 * bound(x[m:m + 1], O.dequant(
                        t, blocks, N * K).reshape(N, K)[[got, want]]).max() + 1e-6, (M_, m, got, want)
                # the lowest index of the tied rows, the masked one skipped
                assert int(i[0][v[0] == v[0].max()].min()) == (4300 if mask < 0 else 4321)
    finally:
        ctx.lib.mlg_matrix_free(w)


def test_lm_head_3b3_batch64(ctx):
    """The 3.3B model's batched LM head at its real size: the q6_K token embedding (256206 x
    2048) of the GGUF file bench.py times, 64 rows.  The logits of mlg_gemm (the wide-tile GEMM,
    split-B q6_K slices) on 2048 sampled rows against the oracle's f64 dot (2e-6 of
    sum |x||w|); mlg_gemm_argmax (the same GEMM with the argmax epilogue, row 7 masked)
    against the argmax of those logits, with planted rows that make the winners known: row
    1000 m + 1007 (x[m]'s signs) wins row m once row 7 (the signs of all 64 rows, so it would
    win every row) is masked."""
    from bench import model_path_3b
    from malaga_amd.gguf import tensor_bytes

    N, K, Mr = 256206, 2048, 64
    raw, info = tensor_bytes(model_path_3b("q4_k_m"), "token_embd.weight")
    assert info["type"] == Q6_K and list(info["ne"]) == [K, N]
    blocks = np.array(raw)  # a writable copy
    row_bytes = len(blocks) // N
    rng = np.random.default_rng(77)
    x = rng.normal(0, 1, (Mr, K)).astype(np.float32)
    planted = {1000 * m + 1007: 0.05 * np.sign(x[m]) for m in range(Mr)}
    planted[7] = 0.5 * np.sign(x).sum(0)
    for r, v in planted.items():
        blocks[r * row_bytes:(r + 1) * row_bytes] = M.quantize(Q6_K, v.astype(np.float32)[None])
    w = upload(ctx, Q6_K, blocks, N, K)
    try:
        xd = dev(x)
        y = torch.empty((Mr, N), device="cuda")
        _lib.check(ctx.lib.mlg_gemm(w, ptr(xd), Mr, ptr(y), None, 0, None))
        torch.cuda.synchronize()
        rows = np.sort(rng.choice(N, 2048, replace=False))
        rows[:2] = (7, 63007)
        rows = np.unique(rows)
        sub = np.ascontiguousarray(blocks.reshape(N, row_bytes)[rows]).reshape(-1)
        ref = O.gemv(Q6_K, sub, len(rows), K, x)
        wd = O.dequant(Q6_K, sub, len(rows) * K).reshape(len(rows), K)
        yl = y.cpu().numpy()
        assert (np.abs(yl[:, rows] - ref) <= 2e-6 * bound(x, wd) + 1e-6).all()
        win = 1000 * np.arange(Mr) + 1007
        assert (yl[:, 7] > yl[np.arange(Mr), win]).all()  # row 7 would win: the mask matters
        parts = ctx.lib.mlg_gemm_argmax_parts(w, Mr)
        assert parts > 0
        pv = torch.zeros((Mr, parts), device="cuda")
        pi = torch.zeros((Mr, parts), dtype=torch.int32, device="cuda")
        _lib.check(ctx.lib.mlg_gemm_argmax(w, ptr(xd), Mr, 7, ptr(pv), ptr(pi), None))
        torch.cuda.synchronize()
        v, i = pv.cpu().numpy(), pi.cpu().numpy().view(np.uint32)
        yl[:, 7] = -np.inf
        for m in range(Mr):
            best = v[m].max()
            got = int(i[m][v[m] == best].min())
            assert got == win[m] == int(np.argmax(yl[m])), (m, got)
            assert best == yl[m, got]  # the same GEMM arithmetic: the same value bit for bit
    finally:
        ctx.lib.mlg_matrix_free(w)


@pytest.mark.parametrize("t,K,N", [(Q4_K, 1024, 70001), (Q5_K, 512, 70001), (Q6_K, 1024, 70001), (Q6_K, 2048, 70001),
                                   (Q6_K, 256, 70001), (Q8_0, 1024, 70001), (Q8_0, 96, 70001),
                                   # the LM head at BASELINE config 2's full size: 256206 x 1024
                                   (Q4_K, 1024, 256206), (Q8_0, 1024, 256206), (Q6_K, 1024, 256206)])
def test_large_gemv_integer_limbs(ctx, t, K, N):
    """N > 65536: the streaming GEMVs hold x as 8-bit limbs with one power-of-two
    scale per group (exact integer dot products).  Besides f32 rounding, each x_k
    is rounded by at most 2^-23 of its group's max |x|; the store and the fused
    argmax (LM head) both follow the dequantized f64 dot product.  q6_K matrices
    read the lane-major copy of their quants (K = 2048: two chunks per lane).  At
    N = 256206 the launch is one resident round of workgroups and the rows past the
    first 32 MB are loaded non-temporally."""
    rng = np.random.default_rng(K + t + N)
    wf = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    blocks = M.quantize(t, wf)
    w = upload(ctx, t, blocks, N, K)
    try:
        wd = O.dequant(t, blocks, N * K).reshape(N, K)
        absw = np.abs(wd.astype(np.float64)).sum(1)
        for b in sorted({1, ctx.lib.mlg_gemv_max_batch(w)}):
            x = rng.normal(0, 1, (b, K)).astype(np.float32)
            x[:, 5] = 40.0  # a group whose scale is set by one large value
            ref = O.gemv(t, blocks, N, K, x)
            tol = 2e-6 * bound(x, wd) + 2.0 ** -22 * np.abs(x).max(1, keepdims=True) * absw + 1e-6
            xd, yd = dev(x), torch.zeros((b, N), device="cuda")
            _lib.check(ctx.lib.mlg_gemv(w, ptr(xd), b, ptr(yd), None, 0, None))
            torch.cuda.synchronize()
            err = np.abs(yd.cpu().numpy() - ref)
            assert (err <= tol).all(), (b, err.max())
            parts = ctx.lib.mlg_gemv_argmax_parts(w, b)
            pv = torch.zeros((b, parts), device="cuda")
            pi = torch.zeros((b, parts), dtype=torch.int32, device="cuda")
            _lib.check(ctx.lib.mlg_gemv_argmax(w, ptr(xd), b, -1, ptr(pv), ptr(pi), None))
            torch.cuda.synchronize()
            v, i = pv.cpu().numpy(), pi.cpu().numpy().view(np.uint32)
            for r in range(b):
                top = np.argsort(ref[r])[::-1][:2]
                k = int(np.argmax(v[r]))
                assert abs(v[r][k] - ref[r][top[0]]) <= tol[r][top[0]]
                if ref[r][top[0]] - ref[r][top[1]] > 2 * tol[r].max():
                    assert i[r][k] == top[0]
    finally:
        ctx.lib.mlg_matrix_free(w)


@pytest.mark.parametrize("t", [Q6_K, Q4_K, Q8_0])
def test_gemv_argmax_lowest_index_on_ties(ctx, t):
    rng = np.random.default_rng(99)
    N, K = 20000, 1024
    wf = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    wf[7777] = wf[12345] = wf[19999] = wf[3] * 0 + rng.normal(0, 0.5, K).astype(np.float32)  # dominant, tied rows
    blocks = M.quantize(t, wf)
    w = upload(ctx, t, blocks, N, K)
    try:
        b = ctx.lib.mlg_gemv_max_batch(w)
        x = np.tile(np.abs(rng.normal(0, 1, K)).astype(np.float32) * np.sign(wf[7777]), (b, 1))
        parts = ctx.lib.mlg_gemv_argmax_parts(w, b)
        xd = dev(x)
        pv = torch.zeros((b, parts), device="cuda")
        pi = torch.zeros((b, parts), dtype=torch.int32, device="cuda")
        _lib.check(ctx.lib.mlg_gemv_argmax(w, ptr(xd), b, -1, ptr(pv), ptr(pi), None))
        torch.cuda.synchronize()
        v, i = pv.cpu().numpy(), pi.cpu().numpy().view(np.uint32)
        for r in range(b):
            k = np.argmax(v[r])  # first max over parts; parts cover increasing row ranges
            best = v[r].max()
            assert i[r][v[r] == best].min() == 7777
        # mask the winner's index: the next tied row wins
        _lib.check(ctx.lib.mlg_gemv_argmax(w, ptr(xd), b, 7777, ptr(pv), ptr(pi), None))
        torch.cuda.synchronize()
        v, i = pv.cpu().numpy(), pi.cpu().numpy().view(np.uint32)
        assert i[0][v[0] == v[0].max()].min() == 12345
    finally:
        ctx.lib.mlg_matrix_free(w)


def test_residual_layernorm(ctx):
    """One wave per row (rows need not fill the four waves of a workgroup), rows up to
    4096 wide; x += y is stored exactly, h follows the f64 LayerNorm."""
    rng = np.random.default_rng(1)
    for rows, d in ((1, 1024), (5, 2048), (3, 64), (7, 4096), (4, 256), (9, 1000)):
        x = rng.normal(0, 3, (rows, d)).astype(np.float32)
        y = rng.normal(0, 1, (rows, d)).astype(np.float32)
        g = rng.normal(1, 0.1, d).astype(np.float32)
        b = rng.normal(0, 0.1, d).astype(np.float32)
        xd, yd, gd, bd, hd = dev(x), dev(y), dev(g), dev(b), torch.zeros((rows, d), device="cuda")
        _lib.check(ctx.lib.mlg_residual_ln(ptr(xd), ptr(yd), rows, d, ptr(gd), ptr(bd), C.c_float(1e-5), ptr(hd), None))
        torch.cuda.synchronize()
        s = x.astype(np.float64) + y
        np.testing.assert_allclose(xd.cpu().numpy(), (x + y), rtol=0, atol=0)
        mu, var = s.mean(1, keepdims=True), s.var(1, keepdims=True)
        ref = (s - mu) / np.sqrt(var + 1e-5) * g + b
        np.testing.assert_allclose(hd.cpu().numpy(), ref, atol=2e-5, rtol=0)
        # LayerNorm alone (encoder input, final norms)
        od = torch.zeros((rows, d), device="cuda")
        _lib.check(ctx.lib.mlg_layernorm(ptr(xd), rows, d, ptr(gd), ptr(bd), C.c_float(1e-5), ptr(od), None))
        torch.cuda.synchronize()
        np.testing.assert_allclose(od.cpu().numpy(), ref, atol=2e-5, rtol=0)


@pytest.mark.parametrize("hd", [8, 16, 32, 64, 128, 256])
def test_attention_decode(ctx, hd):
    """One wave per (row, head) for every supported head size; keys split over lane
    groups with an online softmax; cross lengths and the self-attention step counter."""
    rng = np.random.default_rng(2 + hd)
    b, H, L = 3, 1024 // hd if hd <= 64 else 8, 100
    q = (rng.normal(0, 1, (b, H, hd)) / np.sqrt(hd)).astype(np.float32)  # pre-scaled, as W_q is
    K = rng.normal(0, 1, (b, H, L, hd)).astype(np.float16)
    V = rng.normal(0, 1, (b, H, L, hd)).astype(np.float16)
    lens = np.array([1, 37, 100], dtype=np.uint32)
    qd, kd, vd, ld, od = dev(q), dev(K), dev(V), dev(lens.view(np.int32)), torch.zeros((b, H * hd), device="cuda")
    _lib.check(ctx.lib.mlg_attn_decode(ptr(qd), ptr(kd), ptr(vd), b, H, hd, L, ptr(ld), None, ptr(od), None))
    torch.cuda.synchronize()
    out = od.cpu().numpy().reshape(b, H, hd)
    for i in range(b):
        n = lens[i]
        s = np.einsum("hd,hld->hl", q[i].astype(np.float64), K[i, :, :n].astype(np.float64))
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        ref = np.einsum("hl,hld->hd", p, V[i, :, :n].astype(np.float64))
        np.testing.assert_allclose(out[i], ref, atol=2e-5, rtol=0)
    # self-attention length from the device step counter: n = step + 1
    step = dev(np.array([36], dtype=np.int32))
    _lib.check(ctx.lib.mlg_attn_decode(ptr(qd), ptr(kd), ptr(vd), b, H, hd, L, None, ptr(step), ptr(od), None))
    torch.cuda.synchronize()
    np.testing.assert_allclose(od.cpu().numpy().reshape(b, H, hd)[1], out[1], atol=1e-6)


def test_argmax_partial_full_vocabulary(ctx):
    """BASELINE config 2's argmax over 256206 f32 logits (kernels/malaga.cu:247-280 then
    the merge): the partial maxima merge to np.argmax's answer, ties go to the lowest
    index, and the masked id is never chosen."""
    rng = np.random.default_rng(4)
    b, V = 4, 256206
    x = rng.normal(0, 1, (b, V)).astype(np.float32)
    x[1, 200000] = x[1, 9] = 11.0  # tie across partials: 9 wins
    x[2, V - 1] = 12.0  # the last id
    x[3, 2] = 50.0  # masked below: the runner-up wins
    xd = dev(x)
    for parts in (1, 64, 300):
        pv = torch.zeros((b, parts), device="cuda")
        pi = torch.zeros((b, parts), dtype=torch.int32, device="cuda")
        for mask in (-1, 2):
            _lib.check(ctx.lib.mlg_argmax_partial(ptr(xd), b, V, mask, ptr(pv), ptr(pi), parts, None))
            torch.cuda.synchronize()
            v, i = pv.cpu().numpy(), pi.cpu().numpy().view(np.uint32)
            ref = x.copy()
            if mask >= 0:
                ref[:, mask] = -np.inf
            for r in range(b):
                best = v[r].max()
                got = int(i[r][v[r] == best].min())
                assert got == int(np.argmax(ref[r])), (parts, mask, r)
                assert best == ref[r].max()
            assert int(i[1][v[1] == v[1].max()].min()) == 9


def test_logsoftmax_topk(ctx):
    rng = np.random.default_rng(3)
    rows, V, k = 6, 256206, 4
    x = rng.normal(0, 1, (rows, V)).astype(np.float32)
    x[2, 100] = x[2, 50] = x[2, 7000] = 9.0  # ties -> lowest index first
    x[3, 10:60] = 8.5  # 50 equal values inside one workgroup's chunk, over many threads' lists
    xd = dev(x)
    scratch = torch.zeros(ctx.lib.mlg_logsoftmax_topk_scratch(rows, k) // 4 + 1, device="cuda")
    vals = torch.zeros((rows, k), device="cuda")
    idx = torch.zeros((rows, k), dtype=torch.int32, device="cuda")
    for mask in (-1, 2):
        _lib.check(ctx.lib.mlg_logsoftmax_topk(ptr(xd), rows, V, k, mask, ptr(scratch), ptr(vals), ptr(idx), None))
        torch.cuda.synchronize()
        xx = x.astype(np.float64).copy()
        if mask >= 0:
            xx[:, mask] = -np.inf
        lse = np.log(np.exp(xx - xx.max(1, keepdims=True)).sum(1)) + xx.max(1)
        order = np.lexsort((np.tile(np.arange(V), (rows, 1)), -xx), axis=1)[:, :k]
        np.testing.assert_array_equal(idx.cpu().numpy(), order)
        np.testing.assert_allclose(vals.cpu().numpy(), np.take_along_axis(xx, order, 1) - lse[:, None], atol=2e-5)
    assert idx.cpu().numpy()[2, :3].tolist() == [50, 100, 7000]
    assert idx.cpu().numpy()[3].tolist() == [10, 11, 12, 13]


def test_attention_rejects_unsupported_head_size(ctx):
    q = torch.zeros(1, 48, device="cuda")
    kv = torch.zeros(1, 1, 4, 48, dtype=torch.float16, device="cuda")
    o = torch.zeros(1, 48, device="cuda")
    lens = dev(np.array([4], dtype=np.int32))
    st = ctx.lib.mlg_attn_decode(ptr(q), ptr(kv), ptr(kv), 1, 1, 48, 4, ptr(lens), None, ptr(o), None)
    assert st != 0


def test_greedy_finalize_bookkeeping(ctx):
    """kernels/malaga.cu:290-326: tok = finished ? pad : argmax; finished |= tok == eos; out[:, step]; ++step."""
    b, P, m = 4, 8, 10
    pv = np.full((b, P), -1.0, np.float32)
    pi = np.zeros((b, P), np.uint32)
    pv[0, 3], pi[0, 3] = 5.0, 42
    pv[1, 2], pi[1, 2] = 5.0, 2      # eos
    pv[2, 1], pi[2, 1] = 7.0, 9
    pv[2, 5], pi[2, 5] = 7.0, 8      # tie -> lower index 8
    pv[3, 0], pi[3, 0] = 1.0, 77     # already finished -> pad
    fin = np.array([0, 0, 0, 1], np.uint8)
    pvd, pid, find = dev(pv), dev(pi.view(np.int32)), dev(fin)
    ids = torch.zeros(b, dtype=torch.int32, device="cuda")
    out = torch.zeros((b, m), dtype=torch.int32, device="cuda")
    step = dev(np.array([3], np.int32))
    _lib.check(ctx.lib.mlg_greedy_finalize(ptr(pvd), ptr(pid), P, b, ptr(find), ptr(ids), ptr(out), m, ptr(step),
                                           2, 1, None))
    torch.cuda.synchronize()
    assert ids.cpu().tolist() == [42, 2, 8, 1]
    assert out.cpu().numpy()[:, 3].tolist() == [42, 2, 8, 1]
    assert find.cpu().tolist() == [0, 1, 0, 1]
    assert step.cpu().tolist() == [4]


@pytest.mark.parametrize("b,P", [(5, 7), (17, 1001), (33, 1100), (47, 2100), (64, 1001)])
def test_greedy_finalize_batched(ctx, b, P):
    """The batched finalize (b > 4: two rows per pass, 1024 partials per pass and row):
    lowest index among equal maxima, also across passes, EOS and finished rows, against a
    numpy restatement of kernels/malaga.cu:290-326."""
    rng = np.random.default_rng(b * 1000 + P)
    m, eos, pad, s0 = 12, 2, 1, 5
    pv = rng.normal(0, 1, (b, P)).astype(np.float32)
    pi = rng.permutation(b * P).reshape(b, P).astype(np.uint32) + 10
    for r in range(b):  # a planted maximum, tied in a later (or earlier) partial with a lower index
        j1, j2 = rng.integers(0, P, 2)
        pv[r, j1] = pv[r, j2] = 9.0 + (r % 3)
        pi[r, j2] = min(pi[r, j1], pi[r, j2]) - 1 if r % 2 else pi[r, j2]
    pv[3, -1], pi[3, -1] = 50.0, eos          # row 3 picks EOS from the very last partial
    fin = (rng.random(b) < 0.2).astype(np.uint8)
    fin[3] = 0
    want = []
    for r in range(b):
        mx = pv[r].max()
        tok = int(pi[r][pv[r] == mx].min())
        want.append(pad if fin[r] else tok)
    want_fin = [1 if (fin[r] or want[r] == eos) else 0 for r in range(b)]
    pvd, pid, find = dev(pv), dev(pi.view(np.int32)), dev(fin)
    ids = torch.zeros(b, dtype=torch.int32, device="cuda")
    out = torch.zeros((b, m), dtype=torch.int32, device="cuda")
    step = dev(np.array([s0], np.int32))
    _lib.check(ctx.lib.mlg_greedy_finalize(ptr(pvd), ptr(pid), P, b, ptr(find), ptr(ids), ptr(out), m, ptr(step),
                                           eos, pad, None))
    torch.cuda.synchronize()
    assert ids.cpu().tolist() == want
    assert out.cpu().numpy()[:, s0].tolist() == want
    assert find.cpu().tolist() == want_fin
    assert step.cpu().tolist() == [s0 + 1]
