"""Parity of the gfx950 Q4_K GEMV and activation quantiser against the CPU
oracle (or_quant_q8 restating quant_kernel, src/kernel/q4k_gemv.cu:9-33;
or_gemv_q4k: the dequantised product in double, the value gemv_kernel
q4k_gemv.cu:35-91 computes in fp32).

Quantisation is bit-exact (IEEE divide and round-to-nearest-even on both
sides).  The GEMV sums in fp32 in its own order: the tolerance is 2e-6 of the
row's sum of |terms| (the reference's own self-test allows 1e-5 of one block,
tests/selftest_q4k.cpp:72-74)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def random_blocks(rng, rows, cols):
    b = rng.integers(0, 256, (rows, cols // 256, 144), dtype=np.uint8)
    b[..., 0:2] = rng.uniform(2e-4, 4e-3, (rows, cols // 256, 1)).astype(np.float16).view(np.uint8)
    b[..., 2:4] = rng.uniform(1e-4, 2e-3, (rows, cols // 256, 1)).astype(np.float16).view(np.uint8)
    return b


def abs_terms(oracle, w, rows, cols, qs, d):
    """sum over k of |w_rk * x_k| (dequantised), for the tolerance"""
    out = np.empty(rows)
    xq = np.abs(qs[0].astype(np.float64) * np.repeat(d[0].astype(np.float64), 32))
    for r in range(rows):
        y = np.concatenate([oracle.q4k_dequant_block(w[r, b]) for b in range(cols // 256)]).astype(np.float64)
        out[r] = np.abs(y) @ xq
    return out


@pytest.mark.parametrize("rows,cols", [(3, 3584), (1, 18944), (2, 256), (4, 32768)])
def test_quant_bit_exact(rows, cols, nova7, oracle):
    nova = nova7
    print(f"[case] quant rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(cols + rows)
    x = (rng.standard_normal((rows, cols)) * rng.uniform(0.01, 20, (rows, 1))).astype(np.float32)
    x[0, 64:96] = 0.0                                          # an all-zero block
    dx = nova.upload(x)
    qs, d, s = nova.alloc(rows * cols), nova.alloc(rows * cols // 8), nova.alloc(rows * cols // 4)
    nova.launch_quant_q8(qs.ptr, d.ptr, s.ptr, dx.ptr, rows, cols, None)
    nova.dev_sync()
    rq, rd, rs = oracle.quant_q8(x)
    assert np.array_equal(qs.numpy((rows, cols), np.int8), rq)
    assert np.array_equal(d.numpy((rows, cols // 32), np.float32), rd)
    assert np.array_equal(s.numpy((rows, cols // 16), np.int32), rs)


@pytest.mark.parametrize("rows,cols", [(37, 256), (20, 1536), (512, 3584), (3584, 3584), (50, 5120), (11, 8192),
                                       (70, 8960), (33, 13824), (130, 18944), (9, 32768), (1000, 2560),
                                       (1, 3584), (3, 18944)])
def test_gemv_matches_oracle(rows, cols, nova7, oracle):
    nova = nova7
    print(f"[case] gemv rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    w = random_blocks(rng, rows, cols)
    x = rng.standard_normal((1, cols)).astype(np.float32)
    qs, d, s = oracle.quant_q8(x)
    dw, dq, dd, ds = nova.upload(w), nova.upload(qs), nova.upload(d), nova.upload(s)
    out = nova.upload(np.full(rows, np.nan, np.float32))
    nova.launch_gemv_q4k(dw.ptr, rows, cols, dq.ptr, dd.ptr, ds.ptr, out.ptr, None)
    nova.dev_sync()
    got = out.numpy((rows,), np.float32).astype(np.float64)
    ref = oracle.gemv_q4k(w, rows, cols, qs, d, s)
    check = slice(None) if rows <= 600 else slice(0, rows, max(rows // 300, 1))
    scale = abs_terms(oracle, w[check], len(range(rows)[check]), cols, qs, d)
    err = np.abs(got[check] - ref[check])
    assert np.all(np.isfinite(got))
    assert np.all(err <= 2e-6 * scale), f"max err/scale {np.max(err / scale):.2e}"
    print(f"  max |gpu-oracle| / sum|terms| = {np.max(err / scale):.2e}")


@pytest.mark.parametrize("cols,rows", [(3584, (37, 0, 512)), (3584, (3584,)), (18944, (130, 61)), (256, (5, 1, 2, 9)),
                                       (8960, (33, 70)), (32768, (3, 4))])
def test_gemv_f32_fused(cols, rows, nova7, oracle):
    """launch_gemv_q4k_f32 (quantise inside the launch, up to 4 matrices over one
    activation) equals launch_quant_q8 + launch_gemv_q4k per matrix bit for
    bit, and the oracle within the GEMV tolerance."""
    import ctypes as C
    nova = nova7
    print(f"[case] gemv f32 fused cols={cols} rows={rows}", flush=True)
    rng = np.random.default_rng(cols + sum(rows))
    ws = [random_blocks(rng, r, cols) for r in rows]
    x = (rng.standard_normal((1, cols)) * rng.uniform(0.1, 8.0)).astype(np.float32)
    x[0, 64:96] = 0.0                                      # an all-zero 32-block: d = 0
    dx = nova.upload(x)
    dws = [nova.upload(w) if w.size else nova.alloc(16) for w in ws]
    fused = [nova.upload(np.full(max(r, 1), np.nan, np.float32)) for r in rows]
    sep = [nova.upload(np.full(max(r, 1), np.nan, np.float32)) for r in rows]
    n = len(rows)
    bl = (C.c_void_p * n)(*[d.ptr for d in dws])
    rw = (C.c_int64 * n)(*rows)
    ou = (C.c_void_p * n)(*[o.ptr for o in fused])
    nova.launch_gemv_q4k_f32(bl, rw, ou, n, cols, dx.ptr, None)
    qs, dd, ss = nova.alloc(cols), nova.alloc(cols // 8), nova.alloc(cols // 4)
    nova.launch_quant_q8(qs.ptr, dd.ptr, ss.ptr, dx.ptr, 1, cols, None)
    for m, r in enumerate(rows):
        nova.launch_gemv_q4k(dws[m].ptr, r, cols, qs.ptr, dd.ptr, ss.ptr, sep[m].ptr, None)
    nova.dev_sync()
    oq, od, os_ = oracle.quant_q8(x)
    for m, r in enumerate(rows):
        if r == 0:
            assert np.isnan(fused[m].numpy((1,), np.float32)[0])       # nothing written
            continue
        got = fused[m].numpy((r,), np.float32)
        assert np.array_equal(got.view(np.uint32), sep[m].numpy((r,), np.float32).view(np.uint32)), m
        check = slice(None) if r <= 600 else slice(0, r, max(r // 300, 1))
        ref = oracle.gemv_q4k(ws[m], r, cols, oq, od, os_)
        scale = abs_terms(oracle, ws[m][check], len(range(r)[check]), cols, oq, od)
        err = np.abs(got[check].astype(np.float64) - ref[check])
        assert np.all(err <= 2e-6 * scale), f"matrix {m}: max err/scale {np.max(err / scale):.2e}"


@pytest.mark.parametrize("rows,cols", [(37, 256), (512, 3584), (3584, 3584), (130, 18944), (70, 8960),
                                       (33, 13824), (5, 28672), (1, 1536),
                                       # 32M weights and up: the MFMA kernel (ragged 16-row blocks too)
                                       (2051, 16384), (20001, 2048), (18944, 3584), (3584, 18944)])
def test_gemv4_matches_single_token(rows, cols, nova7, oracle):
    """launch_gemv4_q4k (4 stacked tokens, one weight read): every token's
    output within the GEMV tolerance of the oracle, and of launch_gemv_q4k on
    that token (the same terms summed in another order: both kernels are
    within 2e-6 of the row's sum of |terms| of the exact value)."""
    nova = nova7
    print(f"[case] gemv4 rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows * 13 + cols)
    w = random_blocks(rng, rows, cols)
    x = (rng.standard_normal((4, cols)) * rng.uniform(0.2, 5.0, (4, 1))).astype(np.float32)
    x[2, :32] = 0.0
    qs, d, s = oracle.quant_q8(x)
    dw, dq, dd, ds = nova.upload(w), nova.upload(qs), nova.upload(d), nova.upload(s)
    out4 = nova.upload(np.full(4 * rows, np.nan, np.float32))
    nova.launch_gemv4_q4k(dw.ptr, rows, cols, dq.ptr, dd.ptr, ds.ptr, out4.ptr, None)
    singles = []
    for t in range(4):
        o1 = nova.upload(np.full(rows, np.nan, np.float32))
        nova.launch_gemv_q4k(dw.ptr, rows, cols, dq.ptr + t * cols, dd.ptr + t * (cols // 32) * 4,
                             ds.ptr + t * (cols // 16) * 4, o1.ptr, None)
        singles.append(o1)
    nova.dev_sync()
    got = out4.numpy((4, rows), np.float32)
    # every row up to 600, else ~300 spread rows and the last 17 (a ragged last 16-row block)
    check = np.arange(rows) if rows <= 600 else np.unique(np.r_[np.arange(0, rows, rows // 300), np.arange(rows - 17, rows)])
    for t in range(4):
        one = singles[t].numpy((rows,), np.float32)
        ref = oracle.gemv_q4k(w, rows, cols, qs[t:t + 1], d[t:t + 1], s[t:t + 1])
        scale = abs_terms(oracle, w[check], len(check), cols, qs[t:t + 1], d[t:t + 1])
        err = np.abs(got[t][check].astype(np.float64) - ref[check])
        assert np.all(err <= 2e-6 * scale), f"token {t}: max err/scale {np.max(err / scale):.2e}"
        diff = np.abs(got[t][check].astype(np.float64) - one[check])
        assert np.all(diff <= 4e-6 * scale), f"token {t} vs one-token: {np.max(diff / scale):.2e}"
