"""CPU replay of the attention launch plan and of every index the attention kernels compute
(localstack_amd/csrc/forward.hip: attn_plan, attn_kernel, attn1_kernel, attn_rows_kernel, attn_combine_kernel; buffers sized as
model.cpp allocates them), for work-group targets of 512 (the build's; halved for steps of a few tokens in
one row block), 256 and 128, over the shapes the
tests and the benchmark run and past them: every global index stays inside its buffer, every LDS index
inside its array, and the partial rows inside attn_part_rows. No GPU. The replayed plan is held equal to
the library's own (lstk_debug_attn_plan, host code) at the build's target, so the replay cannot drift
from the C++ it checks.

Also a restatement of the kernel's online softmax over 64-cell passes (running max, sum and rescale per
row, P split into fp16 hi + lo parts, passes in which a row sees no cell) against a direct softmax, and of
the chunk combine, so the multi-pass arithmetic is checked on the CPU.
"""
import numpy as np
import pytest

FA_CELLS = 64       # kFaCells
AT_BLOCK = 256      # kAtBlock: 4 wavefronts
MAX_PASSES = 2048   # kAttnMaxPasses: passes per chunk the skip map of many-token steps covers
BLOCK = 256         # kBlock (attn_combine_kernel)
LDS_MAX = 65536
A1_WGS = 256        # kAttn1Wgs: one work-group per CU


def plan(T, n_head, n_kv, n_cells, target=512, rope_in=False, cell_begin=0, hd=128):
    """attn_plan (forward.hip): rows per work-group, row blocks, chunk (cells), chunks; rope_in kept or not.
    The attended cells are [cell_begin, n_cells)."""
    rows = T * (n_head // n_kv)
    rb_rows = 16 if rows <= 16 else 32 if rows <= 32 else 64
    n_rowblk = (rows + rb_rows - 1) // rb_rows
    passes = (n_cells - cell_begin + FA_CELLS - 1) // FA_CELLS
    if rope_in:
        if n_head * passes <= 32768:
            # one pass per chunk; attn1_kernel's chunks (16 cells per wavefront, 4 to 6 wavefronts) widen
            # to 80 or 96 cells when that keeps the launch within 256 work-groups and 64 would not
            cells, chunk = n_cells - cell_begin, FA_CELLS
            if hd == 128 and n_head // n_kv <= 16 and n_kv * passes > A1_WGS:
                for nw in (5, 6):
                    if n_kv * -(-cells // (16 * nw)) <= A1_WGS:
                        chunk = 16 * nw
                        break
            return rb_rows, n_rowblk, chunk, -(-cells // chunk), True
        rope_in = False
    if T > 1 and n_rowblk == 1:  # a few tokens in one row block: half the target
        target //= 2
    want = (target + n_kv * n_rowblk - 1) // (n_kv * n_rowblk)
    if T >= 64 and n_kv * n_rowblk >= 256:  # kAttnSkipMinT, kAttnOneChunkWgs: one chunk per row block
        want = 1
    want = max(1, min(want, passes))
    chunk = (passes + want - 1) // want * FA_CELLS
    n_chunk = (n_cells - cell_begin + chunk - 1) // chunk
    return rb_rows, n_rowblk, chunk, n_chunk, rope_in


def part_rows(n_batch, n_head):
    return 32768 + n_batch * n_head  # attn_part_rows


def check_launch(T, n_head, n_kv, hd, kv_size, n_cells, n_batch, target, rope_in, cell_begin=0):
    """Every access of one attention launch (and its combine) against the buffers' sizes."""
    assert 1 <= T <= n_batch and 1 <= n_cells <= kv_size and kv_size % 32 == 0
    assert 0 <= cell_begin < n_cells and cell_begin % 64 == 0
    grp = n_head // n_kv
    rb_rows, n_rowblk, chunk, n_chunk, rope_in = plan(T, n_head, n_kv, n_cells, target, rope_in, cell_begin, hd)
    NRT = rb_rows // 16
    RB, NK = 16 * NRT, hd // 16
    DT = NK // 4
    rows = T * grp
    if rope_in:  # launch_attn's own condition
        assert T == 1 and rb_rows == 16 and n_rowblk == 1 and grp <= 16
    grid = n_kv * n_chunk * n_rowblk
    wg = np.arange(grid)
    g, rest = wg % n_kv, wg // n_kv
    c, rb = rest % n_chunk, rest // n_chunk
    assert c.max() < n_chunk and rb.max() < n_rowblk and g.max() < n_kv
    begin = cell_begin + c * chunk
    end = np.minimum(begin + chunk, n_cells)
    assert (begin < end).all(), "a chunk without cells"
    assert end.max() == n_cells and begin.min() == cell_begin, "the chunks cover the attended cells"
    row0 = rb * rb_rows
    # s_pos / Q rows: r < rows reads pos[r / grp] and q[(r / grp) * n_head + g * grp + r % grp]
    r = row0[:, None] + np.arange(RB)[None, :]
    on = r < rows
    assert (r[on] // grp < T).all()
    qrow = (r // grp) * n_head + g[:, None] * grp + r % grp
    assert (qrow[on] < T * n_head).all() and (qrow[on] >= 0).all()
    # RoPE prologue: rotated rows r < grp into s_q [16 * hd]
    if rope_in:
        assert grp * hd <= 16 * hd
    # passes: cells c0 .. c0 + 63; V fragments at min(c0 + kc * 16 + 4 lq, kv_size - 4) + 0..3,
    # K fragments and cell tables at min(cell, kv_size - 1)
    last4 = kv_size - 4
    kv_elems = n_kv * (hd // 4) * kv_size * 4
    for b0, e0, gg in zip(begin, end, g):
        c0 = np.arange(b0, e0, FA_CELLS)
        cg = np.minimum(c0[:, None] + (np.arange(4)[:, None] * 16 + 4 * np.arange(4)[None, :]).ravel()[None, :], last4)
        assert cg.min() >= 0 and (cg % 4 == 0).all()
        d = np.arange(hd)
        vi_max = ((gg * (kv_size // 4) + cg.max() // 4) * hd + d.max()) * 4 + 3
        assert vi_max < kv_elems
        cell = c0[:, None] + np.arange(FA_CELLS)[None, :]
        cc = np.minimum(cell, kv_size - 1)
        ki_max = ((gg * (hd // 4) + (hd // 4 - 1)) * kv_size + cc.max()) * 4 + 3
        assert cc.max() < kv_size and ki_max < kv_elems
    skip = T >= 64 and not rope_in
    if rope_in and hd == 128:
        # attn1_kernel<NW> (launch_attn_hd's single-token case, NW = chunk / 16 wavefronts): wavefront w
        # of a work-group runs cells wb = begin + 16 w .. + 15, K of cell min(wb + lr, kv_size - 1); its
        # V fragments and cell-table entries are loads at cv = min(wb + 4 lq, kv_size - 4), 16-byte
        # aligned; LDS: s_q [16][128] f32, s_kv [256] u16, s_o [NW][16][132] f32, s_m / s_l [NW][16] f32
        assert chunk in (64, 80, 96) and grp <= 16
        NW = chunk // 16
        wb = begin[:, None] + 16 * np.arange(NW)[None, :]
        ck = np.minimum(wb[:, :, None] + np.arange(16)[None, None, :], kv_size - 1)
        cv = np.minimum(wb[:, :, None] + 4 * np.arange(4)[None, None, :], kv_size - 4)
        assert ck.min() >= 0 and ck.max() < kv_size
        assert (cv % 4 == 0).all() and cv.min() >= 0 and cv.max() + 3 < kv_size
        lds = 16 * 128 * 4 + 2 * 128 * 2 + NW * 16 * 132 * 4 + 2 * NW * 16 * 4
        assert lds == {4: 43008, 5: 51584, 6: 60160}[NW] and lds <= LDS_MAX  # the compiler's figures
    elif rb_rows == 64 and hd <= 128:
        # attn_rows_kernel: wavefront w fetches K of cell b0 + 16 w + lr, V of cells b0 + 16 w + 4 lq ..
        # + 3 and the cell tables of cell b0 + 16 w + (lane & 15), clamped to the cache; partial rows and
        # outputs are float4 stores at dims 16 dt + 4 lq; LDS: s_k / s_v [4][hd / 16][64] half4, s_cs / s_cp
        # [64] int, s_live [MAX_PASSES] u8 (skip map)
        for b0, e0 in zip(begin, end):
            blocks = np.arange(b0, e0, FA_CELLS)
            assert (blocks % 4 == 0).all()
            wl = 16 * np.arange(4)[:, None] + np.arange(16)[None, :]      # 16 w + lr (or lane & 15)
            ck = np.minimum(blocks[:, None, None] + wl[None], kv_size - 1)
            cv = np.minimum(blocks[:, None, None] + 16 * np.arange(4)[None, :, None] + 4 * np.arange(4)[None, None, :],
                            kv_size - 4)
            assert ck.min() >= 0 and ck.max() < kv_size and (cv % 4 == 0).all() and cv.max() + 3 < kv_size
        assert hd % 4 == 0  # partial rows (hd + 4 floats) and output rows stay 16-byte aligned for the float4 stores
        lds = 2 * 4 * (hd // 16) * 64 * 8 + 2 * 64 * 4 + (MAX_PASSES if skip else 1)
        assert lds <= LDS_MAX
        if hd == 128 and skip:
            assert lds == 35328  # the compiler's figure for attn_rows_kernel<128, true>
    else:
        # LDS of attn_kernel: s_S [RB][64] f32, s_Ph / s_Pl [RB][72] u16, s_M / s_L / s_f [RB], s_pos [RB],
        # s_q [16 hd] (NRT = 1) f32, s_live [MAX_PASSES] u8 (the pass-skipping instantiation of steps of
        # >= 64 tokens)
        lds = (RB * FA_CELLS * 4 + 2 * RB * (FA_CELLS + 8) * 2 + 3 * RB * 4 + RB * 4 + (16 * hd if NRT == 1 else 1) * 4 +
               (MAX_PASSES if skip else 1))
        assert lds <= LDS_MAX
    if skip:  # the skip map holds one byte per pass of the chunk
        assert (chunk + FA_CELLS - 1) // FA_CELLS <= MAX_PASSES
    # outputs: n_chunk == 1 writes out[(t * n_head + h) * hd + d]; else part rows
    if n_chunk > 1:
        t = r // grp
        h = g[:, None] * grp + r % grp
        prow = (t * n_head + h) * n_chunk + c[:, None]
        assert (prow[on] < part_rows(n_batch, n_head)).all()
        assert T * n_head * n_chunk <= part_rows(n_batch, n_head)
        # attn_combine_kernel: grid (n_head, T), LDS [n_chunk rounded to 4] factors + [BLOCK / (hd / 4)][hd]
        clds = (((n_chunk + 3) & ~3) + BLOCK // (hd // 4) * hd) * 4
        assert clds <= LDS_MAX
        assert ((T - 1) * n_head + n_head - 1) * n_chunk + n_chunk - 1 < part_rows(n_batch, n_head)
    return rb_rows, n_rowblk, chunk, n_chunk, rope_in


def test_replayed_plan_is_the_library_plan(lstk):
    """plan() against lstk_debug_attn_plan over the shapes, token counts, cache sizes (multiples of 32 and
    of 256), attended cells and range starts the model can pass."""
    cases = 0
    for n_head, n_kv, hd in SHAPES.values():
        grp = n_head // n_kv
        for kv_size in (96, 288, 1000 // 32 * 32, 1024, 4608, 4352 + 32, 65536, 65600, 131072):
            for n_cells in sorted({min(kv_size, c) for c in (1, 64, 256, 300, 4160, 4352, 5632, 6144, 6200, 8192, 65536, 65600, 131072)}):
                for cell_begin in sorted({0, (n_cells - 1) // 2 // 64 * 64, (n_cells - 1) // 64 * 64}):
                    for T in (1, 2, 8, 32, 64, 256, 512):
                        for rope in ((False, True) if T == 1 and grp <= 16 else (False,)):
                            want = plan(T, n_head, n_kv, n_cells, 512, rope, cell_begin, hd)
                            got = lstk.attn_plan(T, n_head, n_kv, hd, kv_size, n_cells, cell_begin, rope)
                            assert got[:5] == want, (n_head, kv_size, n_cells, cell_begin, T, rope)
                            assert got[5] == n_kv * want[1] * want[3]
                            cases += 1
    assert cases > 1000
    with pytest.raises(lstk.LstkError):
        lstk.attn_plan(1, 32, 4, 128, 1000, 256)  # kv_size not a multiple of 32
    with pytest.raises(lstk.LstkError):
        lstk.attn_plan(1, 32, 4, 128, 1024, 256, cell_begin=32)  # range start not a multiple of 64


SHAPES = {"tiny": (4, 2, 64), "30b": (32, 4, 128), "235b": (64, 4, 128)}
CELLS = [256, 300, 512, 4160, 4352, 5632, 6144, 6200, 8192, 8256, 16384, 32768, 65536, 65600, 131072]


@pytest.mark.parametrize("target", [512, 256, 128])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_every_attention_index_in_bounds(target, shape):
    n_head, n_kv, hd = SHAPES[shape]
    grp = n_head // n_kv
    plans = 0
    for n_cells in CELLS:
        # the cache sizes a model may be made with: multiples of 32 (the cells then end short of a 256 step)
        for kv_size in sorted({(n_cells + 255) // 256 * 256, (n_cells + 31) // 32 * 32}):
            plans += check_cells(n_head, n_kv, hd, grp, n_cells, kv_size, target)
    assert plans > 100


def check_cells(n_head, n_kv, hd, grp, n_cells, kv_size, target):
    """check_launch for every step size and n_batch over n_cells of a kv_size-cell cache, with the range
    from cell 0 and from high in the cache; returns the number of launches checked."""
    plans = 0
    for T in (1, 2, 8, 32, 64, 256, 512):
        for n_batch in sorted({T, 64, 512}):
            if T > n_batch:
                continue
            rope = T == 1 and grp <= 16
            check_launch(T, n_head, n_kv, hd, kv_size, n_cells, n_batch, target, rope)
            plans += 1
            if n_cells > 256:
                # the sequence's lowest block high in the cache: the range starts there
                check_launch(T, n_head, n_kv, hd, kv_size, n_cells, n_batch, target, rope,
                             cell_begin=(n_cells - 256) // 64 * 64)
                plans += 1
    return plans


def test_rope_in_keeps_single_pass_chunks():
    # one token at the 30B shape: one pass per chunk up to 65536 cells, then RoPE leaves the launch; chunks
    # of 80 or 96 cells keep 4097 .. 6144 cells within 256 work-groups
    assert plan(1, 32, 4, 4096, rope_in=True)[2:] == (64, 64, True)
    assert plan(1, 32, 4, 4352, rope_in=True)[2:] == (80, 55, True)
    assert plan(1, 32, 4, 5632, rope_in=True)[2:] == (96, 59, True)
    assert plan(1, 32, 4, 8192, rope_in=True)[2:] == (64, 128, True)
    assert plan(1, 32, 4, 4352, rope_in=True, hd=64)[2:] == (64, 68, True)
    assert plan(1, 32, 4, 65536, rope_in=True)[2:] == (64, 1024, True)
    rb, nrb, chunk, n_chunk, rope = plan(1, 32, 4, 65600, rope_in=True)
    assert not rope and chunk > 64
    # the committed plan without RoPE: several passes per chunk once the target is reached
    assert plan(32, 32, 4, 4352)[2] == 3 * 64
    assert plan(512, 32, 4, 512)[2:4] == (8 * 64, 1)  # a 512-token prompt: 64 row blocks x 4 KV heads, one chunk
    assert plan(64, 32, 4, 4352)[2:4] == (5 * 64, 14)  # 64 tokens: 8 row blocks x 4 KV heads, several chunks


def softmax_passes(s, T_rows, pass_cells=FA_CELLS):
    """The kernel's online softmax for rows of scores s [rows][cells] (-inf = masked) over passes of
    pass_cells: per pass m_new = max(m_old, max s), p = exp(s - m_new) split into fp16 hi + lo, f =
    exp(m_old - m_new) (0 while m_old = -inf), L = L f + sum p, O = O f + (hi + lo) V. Returns
    (m, L, O) per row for V = identity columns (O = the unnormalised weights)."""
    rows, n = s.shape
    m = np.full(rows, -np.inf, np.float32)
    L = np.zeros(rows, np.float32)
    O = np.zeros((rows, n), np.float32)
    for c0 in range(0, n, pass_cells):
        sv = s[:, c0:c0 + pass_cells]
        mx = np.max(sv, axis=1)
        m_new = np.maximum(m, mx)
        with np.errstate(invalid="ignore"):
            p = np.where(sv == -np.inf, 0.0, np.exp(sv - m_new[:, None])).astype(np.float32)
        hi = p.astype(np.float16).astype(np.float32)
        lo = (p - hi).astype(np.float16).astype(np.float32)
        with np.errstate(invalid="ignore"):
            f = np.where(m == -np.inf, 0.0, np.exp(m - m_new)).astype(np.float32)
        L = L * f + p.sum(axis=1, dtype=np.float32)
        O = O * f[:, None]
        O[:, c0:c0 + pass_cells] += hi + lo
        m = m_new
    return m, L, O


def test_online_softmax_over_passes_and_chunks_matches_direct():
    rng = np.random.default_rng(5)
    rows, n = 48, 1024
    s = (rng.standard_normal((rows, n)) * 4).astype(np.float32)
    # causal-like masks, rows that see nothing in early passes, one row that sees a single cell
    for r in range(rows):
        s[r, : (r * 37) % 700] = -np.inf
        s[r, 900 + r:] = -np.inf
    s[0, :] = -np.inf
    s[0, 777] = 1.5
    direct = np.exp(s.astype(np.float64) - np.max(s, axis=1, keepdims=True))
    direct /= direct.sum(axis=1, keepdims=True)
    m, L, O = softmax_passes(s, rows)
    assert np.max(np.abs(O / L[:, None] - direct)) < 2e-6
    assert O[0, 777] / L[0] == 1.0
    # the same scores cut into chunks of 3 passes, each with its own (m, L, O), merged as the combine
    # kernel merges them: out = sum_c O_c e^(m_c - M) / sum_c L_c e^(m_c - M)
    parts = [softmax_passes(s[:, c0:c0 + 192], rows) for c0 in range(0, n, 192)]
    M = np.max([p[0] for p in parts], axis=0)
    fs = [np.where(p[0] == -np.inf, 0.0, np.exp(p[0] - M)) for p in parts]
    Ls = sum(p[1] * f for p, f in zip(parts, fs))
    Os = np.concatenate([p[2] * f[:, None] for p, f in zip(parts, fs)], axis=1)
    assert np.max(np.abs(Os / Ls[:, None] - direct)) < 2e-6


def softmax_wavefronts(s, wave_cells=16, waves=4):
    """attn1_kernel's arithmetic on one 64-cell chunk per row block of cells: each wavefront takes the
    max over its 16 cells, p = e^(s - m_w) in f32, split into fp16 hi + lo (the operand of O^T += V^T P^T),
    and sums p; the four wavefronts' (m_w, l_w, O_w) then merge with factors e^(m_w - M). Returns the
    chunk's (M, L, O) as the partial row the combine reads."""
    rows, n = s.shape
    assert n == wave_cells * waves
    ms, ls, os_ = [], [], []
    for w in range(waves):
        sw = s[:, w * wave_cells:(w + 1) * wave_cells].astype(np.float32)
        m = np.max(sw, axis=1)
        p = np.where(sw == -np.inf, np.float32(0), np.exp(sw - np.where(m == -np.inf, 0, m)[:, None])).astype(np.float32)
        hi = p.astype(np.float16)
        lo = (p - hi.astype(np.float32)).astype(np.float16)
        o = np.zeros((rows, n), np.float64)
        o[:, w * wave_cells:(w + 1) * wave_cells] = hi.astype(np.float64) + lo.astype(np.float64)
        ms.append(m), ls.append(p.sum(axis=1, dtype=np.float32)), os_.append(o)
    M = np.max(ms, axis=0)
    with np.errstate(invalid="ignore"):  # m = M = -inf (no visible cell in the chunk) gives factor 0
        fs = [np.where(m == -np.inf, np.float32(0), np.exp(m - M)) for m in ms]
    return M, sum(l * f for l, f in zip(ls, fs)), sum(o * f[:, None] for o, f in zip(os_, fs))


def test_wavefront_softmax_of_single_token_attention_matches_direct():
    """The single-token kernel's per-wavefront softmax and LDS merge, then the chunk combine, against a
    direct softmax: rows with masked cells, a wavefront with no visible cell, a row that sees one cell."""
    rng = np.random.default_rng(9)
    rows, n = 16, 64 * 12
    s = (rng.standard_normal((rows, n)) * 4).astype(np.float32)
    for r in range(rows):
        s[r, (r * 53) % 400:(r * 53) % 400 + 40] = -np.inf   # whole wavefronts and chunks masked
        s[r, 700 + r:] = -np.inf
    s[3, :] = -np.inf
    s[3, 130] = 0.25
    direct = np.exp(s.astype(np.float64) - np.max(s, axis=1, keepdims=True))
    direct /= direct.sum(axis=1, keepdims=True)
    parts = [softmax_wavefronts(s[:, c0:c0 + 64]) for c0 in range(0, n, 64)]
    M = np.max([p[0] for p in parts], axis=0)
    fs = [np.where(p[0] == -np.inf, 0.0, np.exp(p[0] - M)) for p in parts]
    L = sum(p[1] * f for p, f in zip(parts, fs))
    O = np.concatenate([p[2] * f[:, None] for p, f in zip(parts, fs)], axis=1)
    assert np.max(np.abs(O / L[:, None] - direct)) < 2e-6
    assert O[3, 130] / L[3] == 1.0
    # the restatement catches a combine that leaves out the chunks' factors
    unscaled = np.concatenate([p[2] for p in parts], axis=1)
    assert np.max(np.abs(unscaled / unscaled.sum(axis=1, keepdims=True) - direct)) > 1e-2
