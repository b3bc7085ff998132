"""libvgx's kernels against the oracle, through the C-ABI, on cuda:0.

Bar: bit-exact.  Every output of these kernels is an integer on the q16 grid
(or an fp32 value computed by the same fp32 operations as the oracle), so the
comparisons are equality, including for full-range random weights and
activations where the int32 lanes of the dot products are at their limits.
"""
import numpy as np
import pytest
import torch

import oracle as o
from vgx import mmcf

pytestmark = pytest.mark.gpu

SHAPES = [(768, 768), (384, 768), (2432, 768), (768, 2432), (6400, 768), (1, 64), (7, 32), (33, 96),
          (1536, 768), (1024, 4096)]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def q8_matrix(rng, rows, cols, plane=True, full=False, prebiased=True):
    if full:
        body = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
        m = mmcf.Matrix("q8", rows, cols, body.ravel(), float(rng.uniform(1e-4, 1e-2)), True,
                        rng.uniform(0, 1.2, rows).astype(np.float32) if plane else None)
    else:
        w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
        if plane:
            q, unit, p = mmcf.q8_per_row(w)
        else:
            (q, unit), p = mmcf.q8_from_i16(w), None
        body = (q.view(np.uint8) ^ 0x80).ravel() if prebiased else q.view(np.uint8).ravel()
        m = mmcf.Matrix("q8", rows, cols, body, float(np.float32(unit)), prebiased, p)
    return m


def q4_matrix(rng, rows, cols):
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
    packed, s16, m16, ps, _ = mmcf.q4mat(w)
    return mmcf.Matrix("q4", rows, cols, packed.ravel(), ps, s16=s16.ravel(), m16=m16.ravel())


def t3_matrix(rng, rows, cols):
    lev = rng.integers(-1, 2, (rows, cols)).astype(np.float32)
    w = lev * rng.uniform(0.01, 0.05, (rows, 1)).astype(np.float32)
    packed, unit, plane = mmcf.t3mat(w)
    return mmcf.Matrix("t3", rows, cols, np.frombuffer(packed, np.uint8), unit, plane=plane)


def wsr_of(m):
    if m.kind == "t3":
        return o.row_scales(m.rows, float(np.float32(np.float32(m.scale) * np.float32(127)) * np.float32(m.scale_mul)),
                            m.plane)
    return o.row_scales(m.rows, float(np.float32(m.scale) * np.float32(m.scale_mul)), m.plane)


def oracle_rowval(m, x):
    if m.kind == "q8":
        return o.rowval_q8(m.body, int(m.prebiased), m.rows, m.cols, wsr_of(m), x)
    if m.kind == "q4":
        return o.rowval_q4(m.body, m.s16, m.m16, float(np.float32(m.scale) * np.float32(m.scale_mul)),
                           m.rows, m.cols, x)
    return o.rowval_t3(m.body, m.rows, m.cols, wsr_of(m), x)


def rand_x(rng, n, full=False):
    if full:
        return rng.integers(-32768, 32768, n).astype(np.int16)
    return o.quantize_act(rng.standard_normal(n).astype(np.float32))


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_q8_gemv(gpu, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    for plane, full, pre in ((True, False, True), (False, False, True), (True, True, True), (True, False, False)):
        m = q8_matrix(rng, rows, cols, plane, full, pre)
        W = gpu.upload(m)
        x = rand_x(rng, cols, full)
        res = rand_x(rng, rows)
        v = oracle_rowval(m, x)
        y = host(gpu.matvec(W, dev(x)))
        assert np.array_equal(y, o.store(v)), (plane, full, pre)
        y2 = host(gpu.matvec(W, dev(x), dev(res)))
        assert np.array_equal(y2, o.store(v, res)), (plane, full, pre)


@pytest.mark.parametrize("rows,cols", [(768, 768), (6400, 768), (2432, 768), (33, 96)])
def test_q8_gemv_f32(gpu, rows, cols):
    rng = np.random.default_rng(11)
    m = q8_matrix(rng, rows, cols)
    W = gpu.upload(m)
    xf = rng.standard_normal(cols).astype(np.float32)
    v = oracle_rowval(m, o.quantize_act(xf))
    y = host(gpu.matvec_f32(W, dev(xf)))
    assert np.array_equal(y, o.store_f32(v))


@pytest.mark.parametrize("rows,cols", [(768, 768), (384, 768), (2432, 768), (768, 2432), (6400, 768), (5, 32),
                                       (1024, 4096)])
def test_q4_gemv(gpu, rows, cols):
    rng = np.random.default_rng(rows + 3 * cols)
    m = q4_matrix(rng, rows, cols)
    W = gpu.upload(m)
    for full in (False, True):
        x = rand_x(rng, cols, full)
        res = rand_x(rng, rows)
        v = oracle_rowval(m, x)
        assert np.array_equal(host(gpu.matvec(W, dev(x))), o.store(v))
        assert np.array_equal(host(gpu.matvec(W, dev(x), dev(res))), o.store(v, res))


@pytest.mark.parametrize("rows,cols", [(1024, 1024), (1280, 1024), (4096, 1024), (1024, 4096), (7, 32), (33, 64)])
def test_t3_gemv(gpu, rows, cols):
    rng = np.random.default_rng(rows + 5 * cols)
    m = t3_matrix(rng, rows, cols)
    W = gpu.upload(m)
    for full in (False, True):
        x = rand_x(rng, cols, full)
        res = rand_x(rng, rows)
        v = oracle_rowval(m, x)
        assert np.array_equal(host(gpu.matvec(W, dev(x))), o.store(v))
        assert np.array_equal(host(gpu.matvec(W, dev(x), dev(res))), o.store(v, res))


@pytest.mark.parametrize("rows,cols", [(33, 8), (64, 200), (130, 1000), (7, 40), (36864, 1000)])
def test_t3_columns_multiple_of_8(gpu, rows, cols):
    """t3 rows of any multiple of 8 columns, as the packer pads them
    (engine/tools/mmcf_hf.py:151-156): upload pads each texel row to whole
    32-column chunks of zero codes; the GEMV (decode and, at 36864 rows, the
    four-rows-a-lane plan), the gate, the batched GEMM and the dequantisation
    equal the oracle bit for bit."""
    rng = np.random.default_rng(rows + cols)
    m = t3_matrix(rng, rows, cols)
    W = gpu.upload(m)
    for full in (False, True):
        x = rand_x(rng, cols, full)
        res = rand_x(rng, rows)
        v = oracle_rowval(m, x)
        assert np.array_equal(host(gpu.matvec(W, dev(x))), o.store(v)), full
        assert np.array_equal(host(gpu.matvec(W, dev(x), dev(res))), o.store(v, res)), full
    if rows <= 1000:
        m3 = t3_matrix(rng, rows, cols)
        W3 = gpu.upload(m3)
        x = rand_x(rng, cols)
        assert np.array_equal(host(gpu.ffn_gate(W, W3, dev(x), 1)),
                              o.gate(oracle_rowval(m, x), oracle_rowval(m3, x), 1))
        for ntok in (5, 37):
            xs = np.stack([rand_x(rng, cols) for _ in range(ntok)])
            got = host(gpu.gemm(W, dev(xs)))
            for t in range(ntok):
                assert np.array_equal(got[t], o.store(oracle_rowval(m, xs[t]))), (ntok, t)
        got = host(gpu.dequant(W))
        want = o.dequant_t3(m.body, rows, cols, wsr_of(m))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_t3_columns_refused(gpu):
    from vgx import lib as vl
    rng = np.random.default_rng(5)
    with pytest.raises(vl.VgxError, match="multiple of 8"):
        gpu.upload(t3_matrix(rng, 4, 12))  # the packer pads 12 to 16: not a kernel row length


@pytest.mark.parametrize("kind", ["q8", "q4", "t3"])
def test_dequant_bit_exact(gpu, kind):
    rng = np.random.default_rng(21)
    rows, cols = 70, 128
    m = {"q8": lambda: q8_matrix(rng, rows, cols), "q4": lambda: q4_matrix(rng, rows, cols),
         "t3": lambda: t3_matrix(rng, rows, cols)}[kind]()
    got = host(gpu.dequant(gpu.upload(m)))
    if kind == "q8":
        want = o.dequant_q8(m.body, 1, rows, cols, wsr_of(m))
    elif kind == "q4":
        want = o.dequant_q4(m.body, m.s16, m.m16, m.scale, rows, cols)
    else:
        want = o.dequant_t3(m.body, rows, cols, wsr_of(m))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("kind,rows,cols", [("q8", 2432, 768), ("q4", 2432, 768), ("t3", 4096, 1024),
                                            ("q8", 9, 64)])
def test_ffn_gate(gpu, kind, rows, cols):
    rng = np.random.default_rng(31)
    mk = {"q8": q8_matrix, "q4": q4_matrix, "t3": t3_matrix}[kind]
    m1, m3 = mk(rng, rows, cols), mk(rng, rows, cols)
    W1, W3 = gpu.upload(m1), gpu.upload(m3)
    x = rand_x(rng, cols)
    for hs in (0, 2):
        h = host(gpu.ffn_gate(W1, W3, dev(x), hs))
        assert np.array_equal(h, o.gate(oracle_rowval(m1, x), oracle_rowval(m3, x), hs)), hs


@pytest.mark.parametrize("kind,rows,cols,split", [("q8", 768, 2432, 1216), ("q4", 768, 2432, 1216),
                                                  ("t3", 1024, 4096, 2048), ("q8", 40, 64, 32)])
def test_gemv_add_split(gpu, kind, rows, cols, split):
    rng = np.random.default_rng(41)
    mk = {"q8": q8_matrix, "q4": q4_matrix, "t3": t3_matrix}[kind]
    m = mk(rng, rows, cols)
    m.scale_mul = 4.0  # metadata key 15, k = 2
    W = gpu.upload(m)
    x = rand_x(rng, cols)
    res = rand_x(rng, rows)
    a, b = m.slice_cols(0, split), m.slice_cols(split, cols)
    y1 = o.store(oracle_rowval(a, x[:split]), res)
    want = o.store(oracle_rowval(b, x[split:]), y1)
    assert np.array_equal(host(gpu.matvec_add_split(W, split, dev(x), dev(res))), want)


def test_group_and_logits_argmax(gpu):
    rng = np.random.default_rng(51)
    vocab, dim = 6400, 768
    w = rng.standard_normal((vocab, dim)).astype(np.float32) * 0.02
    tiles = []
    for st in range(0, vocab, mmcf.LOGITS_GRID):
        q, unit, plane = mmcf.q8_per_row(w[st:st + mmcf.LOGITS_GRID])
        tiles.append(mmcf.Matrix("q8", q.shape[0], dim, (q.view(np.uint8) ^ 0x80).ravel(), unit, True, plane))
    g = gpu.group([gpu.upload(t) for t in tiles])
    x = rand_x(rng, dim)
    want = np.concatenate([o.store(oracle_rowval(t, x)) for t in tiles])
    assert np.array_equal(host(g.gemv(dev(x))), want)
    logits, tok = g.logits_argmax(dev(x))
    assert np.array_equal(host(logits), want) and int(host(tok)[0]) == o.argmax_i16(want)
    # ties: the first maximum wins
    xz = np.zeros(dim, np.int16)
    _, tok = g.logits_argmax(dev(xz))
    assert int(host(tok)[0]) == 0
    xf = rng.standard_normal(dim).astype(np.float32)
    wantf = np.concatenate([o.store_f32(oracle_rowval(t, o.quantize_act(xf))) for t in tiles])
    assert np.array_equal(host(g.gemv_f32(dev(xf))), wantf)


# rows held in registers up to 2048 values (per-thread elements <= 8), reread
# above; 33 and 100 leave the last slices short
@pytest.mark.parametrize("dim", [768, 1024, 64, 100, 33, 2048, 2049, 4096])
def test_rmsnorm(gpu, dim):
    rng = np.random.default_rng(dim)
    for scale in (256, 4000):
        x = np.clip(rng.standard_normal(dim) * scale, -32768, 32767).astype(np.int16)
        w = o.quantize_act(rng.uniform(0.5, 1.5, dim).astype(np.float32))
        for eps in (1e-5, 1e-6):
            assert np.array_equal(host(gpu.rmsnorm(dev(x), dev(w), eps)), o.rmsnorm(x, w, eps))
    xs = np.clip(rng.standard_normal((3, dim)) * 3000, -32768, 32767).astype(np.int16)
    xs[1, :] = 32767
    got = host(gpu.rmsnorm_batch(dev(xs), dev(w), 1e-5))
    for t in range(3):
        assert np.array_equal(got[t], o.rmsnorm(xs[t], w, 1e-5)), t


def _rms_case(rng, dim, scale):
    x = np.clip(rng.standard_normal(dim) * scale, -32768, 32767).astype(np.int16)
    w = o.quantize_act(rng.uniform(0.5, 1.5, dim).astype(np.float32))
    return x, w


@pytest.mark.parametrize("kind,rows,cols", [("q8", 768, 768), ("q8", 2432, 768), ("q4", 1536, 768),
                                            ("t3", 1024, 1024), ("q8", 7, 32), ("t3", 33, 96)])
def test_gemv_rms(gpu, kind, rows, cols):
    # rmsnorm then the GEMV in one launch == the two oracle functions in turn
    rng = np.random.default_rng(rows * 7 + cols)
    mk = {"q8": q8_matrix, "q4": q4_matrix, "t3": t3_matrix}[kind]
    m = mk(rng, rows, cols)
    W = gpu.upload(m)
    for scale, eps in ((256, 1e-5), (4000, 1e-6), (3, 1e-5)):
        x, w = _rms_case(rng, cols, scale)
        xn = o.rmsnorm(x, w, eps)
        res = rand_x(rng, rows)
        assert np.array_equal(host(gpu.matvec_rms(W, dev(x), dev(w), eps)), o.store(oracle_rowval(m, xn)))
        got = host(gpu.matvec_rms(W, dev(x), dev(w), eps, res=dev(res)))
        assert np.array_equal(got, o.store(oracle_rowval(m, xn), res)), (scale, eps)


@pytest.mark.parametrize("kind,rows,cols", [("q8", 2432, 768), ("q4", 2432, 768), ("t3", 512, 1024)])
def test_ffn_gate_rms(gpu, kind, rows, cols):
    rng = np.random.default_rng(71)
    mk = {"q8": q8_matrix, "q4": q4_matrix, "t3": t3_matrix}[kind]
    m1, m3 = mk(rng, rows, cols), mk(rng, rows, cols)
    W1, W3 = gpu.upload(m1), gpu.upload(m3)
    x, w = _rms_case(rng, cols, 900)
    xn = o.rmsnorm(x, w, 1e-5)
    for hs in (0, 1):
        h = host(gpu.ffn_gate_rms(W1, W3, dev(x), dev(w), 1e-5, hs))
        assert np.array_equal(h, o.gate(oracle_rowval(m1, xn), oracle_rowval(m3, xn), hs)), hs


@pytest.mark.parametrize("tile", [mmcf.LOGITS_GRID, 600])
def test_logits_argmax_rms(gpu, tile):
    # the final norm, the LM head and the argmax in one launch; tile 600 gives
    # 11 matrices, more than the launch carries by value
    rng = np.random.default_rng(81 + tile)
    vocab, dim = 6400, 768
    wh = rng.standard_normal((vocab, dim)).astype(np.float32) * 0.02
    tiles = []
    for st in range(0, vocab, tile):
        q, unit, plane = mmcf.q8_per_row(wh[st:st + tile])
        tiles.append(mmcf.Matrix("q8", q.shape[0], dim, (q.view(np.uint8) ^ 0x80).ravel(), unit, True, plane))
    g = gpu.group([gpu.upload(t) for t in tiles])
    logits = torch.empty(vocab, dtype=torch.int16, device="cuda")
    token = torch.empty(1, dtype=torch.int32, device="cuda")
    # several launches in a row: the finished-workgroup counter is back at 0
    # after each
    for k in range(4):
        x, w = _rms_case(rng, dim, 300 * (k + 1))
        xn = o.rmsnorm(x, w, 1e-5)
        want = np.concatenate([o.store(oracle_rowval(t, xn)) for t in tiles])
        assert np.array_equal(host(g.gemv_rms(dev(x), dev(w), 1e-5)), want)
        g.logits_argmax_rms(dev(x), dev(w), 1e-5, logits, token)
        assert np.array_equal(host(logits), want)
        assert int(host(token)[0]) == o.argmax_i16(want), k
    # all-zero logits: the first maximum (index 0)
    g.logits_argmax_rms(dev(np.zeros(dim, np.int16)), dev(w), 1e-5, logits, token)
    assert int(host(token)[0]) == 0


def test_logits_argmax_step_matches_separate_launches(gpu):
    # the decode step's tail in the argmax reduction launch: the same token,
    # history, position and next embedding as logits_argmax_rms followed by
    # decode_advance and embed_q8; the next input may be the head's own input
    rng = np.random.default_rng(83)
    vocab, dim = 3000, 256
    wh = rng.standard_normal((vocab, dim)).astype(np.float32) * 0.05
    tiles = []
    for st in range(0, vocab, mmcf.LOGITS_GRID):
        q, unit, plane = mmcf.q8_per_row(wh[st:st + mmcf.LOGITS_GRID])
        tiles.append(mmcf.Matrix("q8", q.shape[0], dim, (q.view(np.uint8) ^ 0x80).ravel(), unit, True, plane))
    g = gpu.group([gpu.upload(t) for t in tiles])
    emb = torch.from_numpy(rng.integers(-128, 128, size=(vocab, dim), dtype=np.int8)).cuda()
    emb_scale = torch.from_numpy(rng.uniform(0.001, 0.05, vocab).astype(np.float32)).cuda()
    hist_len = 16
    for k, p in enumerate((0, 5, hist_len - 2, hist_len - 1)):
        print("argmax step case", k, "pos", p, flush=True)
        x, w = _rms_case(rng, dim, 200 * (k + 1))
        logits = torch.empty(vocab, dtype=torch.int16, device="cuda")
        token = torch.empty(1, dtype=torch.int32, device="cuda")
        g.logits_argmax_rms(dev(x), dev(w), 1e-5, logits, token)
        pos_a = torch.tensor([p], dtype=torch.int32, device="cuda")
        hist_a = torch.arange(hist_len, dtype=torch.int32, device="cuda")
        gpu.decode_advance(pos_a, token, hist_a)
        x_a = gpu.embed_q8(emb, emb_scale, token)
        xb = dev(x)
        logits_b = torch.empty(vocab, dtype=torch.int16, device="cuda")
        token_b = torch.empty(1, dtype=torch.int32, device="cuda")
        pos_b = torch.tensor([p], dtype=torch.int32, device="cuda")
        hist_b = torch.arange(hist_len, dtype=torch.int32, device="cuda")
        g.logits_argmax_step(xb, dev(w), 1e-5, logits_b, token_b, pos_b, hist_b, emb, emb_scale, xb)
        assert np.array_equal(host(logits_b), host(logits))
        assert int(host(token_b)[0]) == int(host(token)[0])
        assert int(host(pos_b)[0]) == int(host(pos_a)[0]) == p + 1
        assert np.array_equal(host(hist_b), host(hist_a))
        assert np.array_equal(host(xb), host(x_a))


def test_rms_entry_point_refusals(gpu):
    rng = np.random.default_rng(91)
    m = q8_matrix(rng, 64, 64)
    W = gpu.upload(m)
    x, w = _rms_case(rng, 64, 256)
    from vgx.lib import VgxError
    with pytest.raises(VgxError):
        gpu.matvec_rms(W, dev(x), dev(w), 0.0)
    with pytest.raises(VgxError):
        gpu.matvec_rms(W, dev(x), dev(w)[1:], 1e-5)  # misaligned weight


def test_embed_q8(gpu):
    rng = np.random.default_rng(61)
    emb = rng.integers(-127, 128, (6400, 768)).astype(np.int8)
    es = rng.uniform(1e-4, 1e-2, 6400).astype(np.float32)
    E, S = dev(emb), dev(es)
    for tok in (0, 17, 6399):
        t = dev(np.array([tok], np.int32))
        assert np.array_equal(host(gpu.embed_q8(E, S, t)), o.embed_q8(emb, es, tok))


def test_mat_clone_and_errors(gpu):
    rng = np.random.default_rng(71)
    m = q8_matrix(rng, 64, 64)
    W = gpu.upload(m)
    C = gpu.clone(W)
    x = dev(rand_x(rng, 64))
    assert torch.equal(gpu.matvec(W, x), gpu.matvec(C, x))
    assert W.weight_bytes == 64 * 64 + 64 * 4
    from vgx import lib as vl
    bad = mmcf.Matrix("q8", 64, 40, np.zeros(64 * 40, np.uint8), 1.0)
    with pytest.raises(vl.VgxError):
        gpu.upload(bad)  # cols not a multiple of 16
    with pytest.raises(vl.VgxError):
        gpu.matvec(W, x[1:])  # misaligned activation pointer


@pytest.mark.parametrize("kind", ["q8", "t3"])
def test_mat_concat_gemm_and_argmax_rows(gpu, kind):
    """The LM head of the batched decode: logits tiles concatenated into one
    matrix keep every row's scale, so its GEMM over n rows equals each tile's
    GEMV on each row; the per-row argmax keeps the first maximum."""
    rng = np.random.default_rng(71)
    dim, sizes = 256, [96, 96, 40]
    tiles = [q8_matrix(rng, r, dim) if kind == "q8" else t3_matrix(rng, r, dim) for r in sizes]
    mats = [gpu.upload(t) for t in tiles]
    cat = gpu.concat(mats)
    assert cat.rows == sum(sizes)
    X = np.stack([rand_x(rng, dim) for _ in range(5)])
    got = host(gpu.gemm(cat, dev(X)))
    for i in range(5):
        want = np.concatenate([o.store(oracle_rowval(t, X[i])) for t in tiles])
        assert np.array_equal(got[i], want), i
    V = rng.integers(-300, 300, (7, 1000)).astype(np.int16)
    V[2, [5, 900]] = 400  # ties: the first maximum wins
    V[4] = 0
    assert np.array_equal(host(gpu.argmax_rows(dev(V))), [o.argmax_i16(v) for v in V])
    from vgx import lib as vl
    with pytest.raises(vl.VgxError):
        gpu.concat([mats[0], gpu.upload(q4_matrix(rng, 32, dim))])  # q4 scales are per matrix
    if kind == "t3":
        odd_t = t3_matrix(rng, 33, dim)
        odd = gpu.upload(odd_t)
        with pytest.raises(vl.VgxError):
            gpu.concat([odd, mats[0]])  # an odd t3 matrix must come last
        cat2 = gpu.concat([mats[0], odd])
        want = np.concatenate([o.store(oracle_rowval(tiles[0], X[0])), o.store(oracle_rowval(odd_t, X[0]))])
        assert np.array_equal(host(gpu.gemm(cat2, dev(X[:1])))[0], want)


# The bandwidth-bound plans: a launch of >= 16 waves per CU takes 4 rows per
# lane, with 16 (q8, K <= 1024) or 8 (q8, K > 1024) lanes a row, and 8 (q4,
# up to 48 groups) or 16 (q4, more) -- the kernels the cold GEMV sweep times.
# Each case is a group of equal-shape copies (one launch) and, where one matrix
# is large enough by itself, a single-matrix launch; both the q16 and the f32
# entry points, bit-exact against the oracle.
BIG = [("q8", 768, 768, 24, (16, 4)), ("q8", 768, 2432, 8, (8, 4)),
       ("q4", 768, 768, 48, (8, 4)), ("q4", 768, 2432, 11, (16, 4))]


@pytest.mark.parametrize("kind,rows,cols,copies,plan", BIG)
def test_gemv_bandwidth_plans(gpu, kind, rows, cols, copies, plan):
    rng = np.random.default_rng(rows + cols + copies)
    mats = [(q8_matrix if kind == "q8" else q4_matrix)(rng, rows, cols) for _ in range(copies)]
    Ws = [gpu.upload(m) for m in mats]
    G = gpu.group(Ws)
    assert G.plan() == plan
    for full in (False, True):
        x = rand_x(rng, cols, full)
        v = np.concatenate([oracle_rowval(m, x) for m in mats])
        assert np.array_equal(host(G.gemv(dev(x))), o.store(v)), full
    xf = rng.standard_normal(cols).astype(np.float32)
    v = np.concatenate([oracle_rowval(m, o.quantize_act(xf)) for m in mats])
    assert np.array_equal(host(G.gemv_f32(dev(xf))), o.store_f32(v))
    G.free()
    # as many rows in one matrix: a single-matrix launch of the same plan
    one = (q8_matrix if kind == "q8" else q4_matrix)(rng, rows * copies, cols)
    W1 = gpu.upload(one)
    assert gpu.plan(W1) == plan
    x = rand_x(rng, cols, True)
    res = rand_x(rng, one.rows)
    v = oracle_rowval(one, x)
    assert np.array_equal(host(gpu.matvec(W1, dev(x), dev(res))), o.store(v, res))
    v = oracle_rowval(one, o.quantize_act(xf))
    assert np.array_equal(host(gpu.matvec_f32(W1, dev(xf))), o.store_f32(v))


def q4_adversarial_matrix(rng, rows, cols):
    from test_oracle_pins import q4_adversarial
    body, s16, m16, ps, _ = q4_adversarial(rng, rows, cols)
    return mmcf.Matrix("q4", rows, cols, body, ps, s16=s16, m16=m16)


# q4 rows whose group terms span ~2^39 (scales of 1-3 beside scales near 2^15,
# minima at the rails, rail and near-empty activation groups): every plan's
# lane order, the gate, the split and the f32 entry point stay bit-exact
@pytest.mark.parametrize("rows,cols,copies,plan", [(768, 768, 1, None), (33, 96, 1, None),
                                                   (768, 768, 48, (8, 4)), (768, 2432, 11, (16, 4))])
def test_q4_adversarial_groups(gpu, rows, cols, copies, plan):
    from test_oracle_pins import q4_adversarial_x
    rng = np.random.default_rng(rows + copies)
    mats = [q4_adversarial_matrix(rng, rows, cols) for _ in range(copies)]
    Ws = [gpu.upload(m) for m in mats]
    x = q4_adversarial_x(rng, cols)
    xf = x.astype(np.float32) / np.float32(256)  # quantize_act gives x back
    assert np.array_equal(o.quantize_act(xf), x)
    v = np.concatenate([oracle_rowval(m, x) for m in mats])
    if copies > 1:
        G = gpu.group(Ws)
        assert G.plan() == plan
        assert np.array_equal(host(G.gemv(dev(x))), o.store(v))
        assert np.array_equal(host(G.gemv_f32(dev(xf))).view(np.uint32), o.store_f32(v).view(np.uint32))
        G.free()
        return
    res = rand_x(rng, rows, True)
    assert np.array_equal(host(gpu.matvec(Ws[0], dev(x), dev(res))), o.store(v, res))
    assert np.array_equal(host(gpu.matvec_f32(Ws[0], dev(xf))).view(np.uint32), o.store_f32(v).view(np.uint32))
    m3 = q4_adversarial_matrix(rng, rows, cols)
    h = host(gpu.ffn_gate(Ws[0], gpu.upload(m3), dev(x), 0))
    assert np.array_equal(h, o.gate(v, oracle_rowval(m3, x), 0))
    split = cols // 2 // 32 * 32
    a, b = mats[0].slice_cols(0, split), mats[0].slice_cols(split, cols)
    y1 = o.store(oracle_rowval(a, x[:split]), res)
    assert np.array_equal(host(gpu.matvec_add_split(Ws[0], split, dev(x), dev(res))),
                          o.store(oracle_rowval(b, x[split:]), y1))


@pytest.mark.parametrize("n", [73448, 6403, 64402, 8])
def test_argmax_rows_first_maximum(gpu, n):
    # 16-byte vectors where a row starts on a 16-byte boundary, the scalar
    # loop for the tail and for unaligned rows (odd n): the first maximum of
    # each row, with ties inside one vector, across lanes and at the ends
    rng = np.random.default_rng(n)
    V = rng.integers(-30000, 30000, (9, n)).astype(np.int16)
    V[0, [n - 1, 0]] = 32767                      # first and last
    V[1, [n // 2, n // 2 + 1]] = 32767            # adjacent (one vector)
    if n > 9000:
        V[2, [8 * 1024 + 3, 3]] = 32767           # another lane's vector first
    if n > 66000:
        V[3, [n - 5, 8 * 1024 * 8 + 1]] = 32767   # a later round
    V[4] = -32768                                 # all equal: index 0
    V[5, -1] = 32767                              # only the tail
    got = host(gpu.argmax_rows(dev(V)))
    assert np.array_equal(got, [o.argmax_i16(v) for v in V])
