// model.cpp - the Qwen3-MoE forward pass around the MoE block (include/lstk_qwen3.h).
//
// lstk_model plays the part of the reference's Engine + qwen3_build_graph + KvCache
// (src/engine.cpp:193-341, src/qwen3.cpp:128-259, src/kv_cache.cpp:59-150) for one GPU and one
// stream. Instead of building a ggml graph per step it launches a fixed kernel sequence:
//   layer 0:  embedding gather + attn_norm             (rmsnorm_kernel; inside the Q/K/V launch at T = 1)
//   each layer l:
//     Q, K, V projections in one launch                 (gemv_kernel, 3 segments; gemv1_kernel at T = 1)
//     QK-norm + NEOX RoPE + K/V store into the cache    (rope_kernel; at T = 1 inside the attention
//                                                        launch)
//     attention over the step's n_kv cells              (attn_kernel [+ attn_combine_kernel])
//     o-proj + residual                                 (gemv_kernel with add)
//     ffn_norm on the rows the FFN needs                (rmsnorm_kernel; at T = 1 with a resident pool
//                                                        the router launch normalises the row itself)
//     MoE block: lstk_moe_block (resident pool) or route -> acquire -> lstk_moe_ffn (streaming pool;
//     the acquire runs on the device for an LSTK_POOL_DEVICE_LRU pool); with several tokens and a
//     resident pool the block's combine + residual is left to the next layer's attn_norm launch,
//     which forms the same sums before it normalises them
//     the last layer runs its FFN on the output row only (src/qwen3.cpp:233-237)
//   output_norm + head on the last row                  (rmsnorm_kernel, gemv_kernel)
// With several tokens per step the projections are plain F16 matrix products: the normalised rows and
// the attention output are also written as fp16 (ggml rounds the activations of an F16 mat-mul to
// fp16) and they are multiplied with f32 accumulation: on the matrix cores by gemm16_kernel (forward.hip)
// up to 16 tokens, by rocBLAS (rocblas_gemm_ex, f16 x f16 -> f32) for more.
// The KV cache keeps the reference's block table (32-cell blocks handed out per sequence, cell_seq /
// cell_pos per cell) on the host; the device holds the cells' fp16 K and V in layouts chosen for
// coalesced reads (forward.h) and a copy of cell_seq / cell_pos that the step's RoPE launch updates.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/lstk_qwen3.h"
#include "forward.h"
#include "internal.h"

namespace {

using lstk::set_error;

constexpr int kStages = 5;
constexpr int kBlasMinTokens = 2; // steps of at least this many tokens take the library GEMM

constexpr uint32_t kCellBlock = 32; // KvCache::block_size (src/kv_cache.h:27)

int hip_fail(hipError_t e, const char *what) { return set_error(LSTK_E_DEVICE, std::string(what) + ": " + hipGetErrorString(e)); }

// The KV cache's cell table (KvCache, src/kv_cache.cpp:59-150). Cells come in blocks of kCellBlock
// that a sequence takes as it grows; position p of a sequence lives in cell
// blocks[p / kCellBlock] * kCellBlock + p % kCellBlock. Spare blocks form a stack whose top starts at
// block 0, and freed blocks are pushed back in the order they are released, so the cell each step
// gets is the reference's. A block holds consecutive positions of one sequence from its first cell,
// so its occupied cells are its first fill[b]; the attended range ends after the last occupied cell.
struct KvBook {
    struct Seq {
        std::vector<uint32_t> blocks;
        int32_t len = 0;
    };
    uint32_t size = 0;
    std::vector<int32_t> cell_seq, cell_pos; // per cell: sequence and position, -1 when free (mirrored to the device)
    std::vector<uint32_t> spare;             // free blocks; the next one handed out is at the back
    std::vector<uint32_t> fill;              // per block: occupied cells
    std::map<int32_t, Seq> seqs;

    void init(uint32_t n) {
        size = n;
        cell_seq.assign(n, -1);
        cell_pos.assign(n, -1);
        const uint32_t nb = n / kCellBlock;
        fill.assign(nb, 0);
        spare.resize(nb);
        for (uint32_t i = 0; i < nb; i++) spare[i] = nb - 1 - i;
        seqs.clear();
    }
    int32_t length(int32_t seq) const {
        const auto it = seqs.find(seq);
        return it == seqs.end() ? 0 : it->second.len;
    }
    uint32_t cell_of(const Seq &q, int32_t p) const { return q.blocks[(uint32_t) p / kCellBlock] * kCellBlock + (uint32_t) p % kCellBlock; }
    void clear_cell(uint32_t c) { cell_seq[c] = cell_pos[c] = -1; }
    bool alloc(int32_t seq, int n, std::vector<int32_t> &cells, std::vector<int32_t> &positions) {
        const bool fresh = seqs.find(seq) == seqs.end();
        Seq &q = seqs[seq];
        const size_t blocks_after = ((size_t) q.len + (size_t) n + kCellBlock - 1) / kCellBlock;
        if (blocks_after > q.blocks.size() + spare.size()) {
            if (fresh) seqs.erase(seq);
            return false;
        }
        while (q.blocks.size() < blocks_after) {
            q.blocks.push_back(spare.back());
            spare.pop_back();
        }
        cells.resize(n);
        positions.resize(n);
        for (int i = 0; i < n; i++) {
            const int32_t p = q.len + i;
            const uint32_t c = cell_of(q, p);
            cell_seq[c] = seq;
            cell_pos[c] = p;
            fill[c / kCellBlock] = c % kCellBlock + 1;
            cells[i] = (int32_t) c;
            positions[i] = p;
        }
        q.len += n;
        return true;
    }
    // Frees the sequence's positions from `keep` on; blocks left empty go back to the spares, last first.
    void shrink(std::map<int32_t, Seq>::iterator it, int32_t keep) {
        Seq &q = it->second;
        for (int32_t p = keep; p < q.len; p++) clear_cell(cell_of(q, p));
        const size_t keep_blocks = ((size_t) keep + kCellBlock - 1) / kCellBlock;
        while (q.blocks.size() > keep_blocks) {
            fill[q.blocks.back()] = 0;
            spare.push_back(q.blocks.back());
            q.blocks.pop_back();
        }
        if (keep_blocks > 0) fill[q.blocks.back()] = (uint32_t) (keep - (int32_t) (keep_blocks - 1) * (int32_t) kCellBlock);
        q.len = keep;
    }
    void remove_seq(int32_t seq) {
        const auto it = seqs.find(seq);
        if (it == seqs.end()) return;
        // every block of the sequence, first to last, back to the spares
        Seq &q = it->second;
        for (uint32_t b : q.blocks) {
            for (uint32_t c = b * kCellBlock; c < b * kCellBlock + fill[b]; c++) clear_cell(c);
            fill[b] = 0;
            spare.push_back(b);
        }
        seqs.erase(it);
    }
    void truncate_seq(int32_t seq, int32_t keep) {
        const auto it = seqs.find(seq);
        if (it == seqs.end()) return;
        if (keep <= 0) return remove_seq(seq);
        if (keep < it->second.len) shrink(it, keep);
    }
    // Engine::n_kv_for (src/engine.cpp:193-196): the cells up to the last occupied one, rounded up to a
    // multiple of 256 (at least 256), capped at the cache size.
    // The first cell of the sequence's lowest block (0 for an unknown sequence): no cell of the sequence
    // lies below it, so the attention need not look there.
    int first_cell(int32_t seq) const {
        const auto it = seqs.find(seq);
        if (it == seqs.end() || it->second.blocks.empty()) return 0;
        return (int) (*std::min_element(it->second.blocks.begin(), it->second.blocks.end()) * kCellBlock);
    }
    int n_kv() const {
        uint32_t end = 0;
        for (uint32_t b = 0; b < (uint32_t) fill.size(); b++)
            if (fill[b] > 0) end = std::max(end, b * kCellBlock + fill[b]);
        const uint32_t padded = (end + 255) / 256 * 256;
        return (int) std::min<uint32_t>(size, std::max<uint32_t>(256, padded));
    }
};

struct TimedLaunch {
    hipEvent_t start = nullptr, end = nullptr;
};

}  // namespace

struct lstk_model {
    lstk_qwen3_hparams hp{};
    std::vector<lstk_qwen3_layer> layers;
    const uint16_t *tok_embd = nullptr, *output = nullptr;
    const float *output_norm = nullptr;
    lstk_pool *pool = nullptr;
    bool streaming = false, device_lru = false;
    int n_batch = 0;
    float theta_scale = 0.0f;
    KvBook kv;
    // device
    void *mem = nullptr;
    uint16_t *kcache = nullptr, *vcache = nullptr;
    size_t layer_elems = 0; // fp16 values of one layer's K (or V) cache
    int32_t *cell_seq = nullptr, *cell_pos = nullptr;
    uint16_t *qr = nullptr; // [n_batch][n_head][head_dim] rotated Q, fp16 (the attention's Q operand)
    float *x = nullptr, *hn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr,
          *part = nullptr, *weights = nullptr;
    int32_t *ids = nullptr, *slots = nullptr, *in = nullptr; // in = tokens | cells | positions
    uint16_t *hn16 = nullptr, *attn16 = nullptr;             // fp16 inputs of the multi-token products
    int ld_qkv = 0; // row stride of q | k | v (one buffer: token t's Q, K and V rows side by side)
    std::vector<char> qkv_joined; // per layer: wk follows wq and wv follows wk in memory
    float *rope_cs = nullptr; // [n_batch][head_dim / 2][2] cos / sin of the step's RoPE angles
    rocblas_handle blas = nullptr;
    // pinned host staging
    int32_t *h_in = nullptr, *h_ids = nullptr, *h_slots = nullptr;
    hipEvent_t in_free = nullptr;
    // timing
    bool timing = false;
    std::vector<TimedLaunch> launched[kStages];
    // test hook: the residual stream after every layer, [n_layer][T][n_embd] (lstk_model_debug_capture)
    float *capture = nullptr;
    // test hook: the residual stream entering every layer's MoE block (lstk_model_debug_capture_moe_in)
    float *capture_moe = nullptr;
    // test hook (lstk_model_debug_options bit 0): RoPE of a single-token step in its own launch
    bool rope_apart = false;
    // routing trace
    FILE *trace = nullptr;
    int32_t *trace_dev = nullptr; // [n_layer][n_batch][k] when the caller passes no trace buffer
    std::vector<int32_t> trace_host;
};

namespace {

template <typename F>
hipError_t timed(lstk_model *M, int stage, F &&launch) {
    if (!M->timing) return launch(nullptr);
    TimedLaunch t{};
    hipError_t e;
    if ((e = hipEventCreate(&t.start)) != hipSuccess) return e;
    if ((e = hipEventCreate(&t.end)) != hipSuccess) return e;
    lstk::LaunchTiming tm;
    tm.start = t.start;
    tm.stop = t.end;
    const hipError_t le = launch(&tm);
    M->launched[stage].push_back(t);
    return le;
}

void destroy(lstk_model *M) {
    if (!M) return;
    if (M->blas) (void) rocblas_destroy_handle(M->blas);
    if (M->trace) fclose(M->trace);
    if (M->trace_dev) (void) hipFree(M->trace_dev);
    if (M->mem) (void) hipFree(M->mem);
    if (M->h_in) (void) hipHostFree(M->h_in);
    if (M->in_free) (void) hipEventDestroy(M->in_free);
    for (auto &v : M->launched)
        for (TimedLaunch &t : v) {
            (void) hipEventDestroy(t.start);
            (void) hipEventDestroy(t.end);
        }
    delete M;
}

int create(const lstk_qwen3_hparams *hpp, const lstk_qwen3_weights *w, lstk_pool *pool, uint32_t kv_size, uint32_t n_batch,
           lstk_model **out) {
    if (!out) return set_error(LSTK_E_INVALID, "out must be non-null");
    *out = nullptr;
    if (!hpp || !w || !pool || !w->layers) return set_error(LSTK_E_INVALID, "null argument");
    const lstk_qwen3_hparams &hp = *hpp;
    if (hp.n_layer < 1 || hp.n_embd < 1 || hp.n_head < 1 || hp.n_head_kv < 1 || hp.head_dim < 1 || hp.n_vocab < 1)
        return set_error(LSTK_E_INVALID, "hyperparameters must be positive");
    if (hp.n_head % hp.n_head_kv) return set_error(LSTK_E_INVALID, "n_head must be a multiple of n_head_kv");
    if (!lstk::attn_supported(hp.head_dim)) return set_error(LSTK_E_INVALID, "head_dim must be 64, 128 or 256");
    if (!lstk::gemv_supported(hp.n_embd) || !lstk::gemv_supported(hp.n_head * hp.head_dim) ||
        !lstk::rmsnorm_supported(hp.n_embd))
        return set_error(LSTK_E_INVALID, "n_embd and n_head * head_dim must be multiples of 8 and at most 8192");
    if (!(hp.rms_eps >= 0.0f) || !(hp.rope_freq_base > 0.0f)) return set_error(LSTK_E_INVALID, "bad rms_eps or rope_freq_base");
    if (kv_size == 0 || kv_size % kCellBlock) return set_error(LSTK_E_INVALID, "kv_size must be a positive multiple of 32");
    if (n_batch == 0) return set_error(LSTK_E_INVALID, "n_batch must be >= 1");
    if (lstk::pool_dry(pool)) return set_error(LSTK_E_INVALID, "the pool was created without device memory");
    const lstk_moe_dims &d = lstk::pool_dims(pool);
    if (d.n_layer != hp.n_layer || d.n_embd != hp.n_embd || d.n_ff_exp != hp.n_ff_exp || d.n_expert != hp.n_expert ||
        d.n_expert_used != hp.n_expert_used)
        return set_error(LSTK_E_INVALID, "the pool's dims do not match the hyperparameters");
    if ((uint32_t) d.n_batch < n_batch) return set_error(LSTK_E_INVALID, "n_batch exceeds the pool's n_batch");
    if (!w->tok_embd || !w->output_norm) return set_error(LSTK_E_INVALID, "tok_embd and output_norm must be non-null");
    for (int l = 0; l < hp.n_layer; l++) {
        const lstk_qwen3_layer &L = w->layers[l];
        if (!L.attn_norm || !L.wq || !L.wk || !L.wv || !L.wo || !L.ffn_norm || !L.gate_inp)
            return set_error(LSTK_E_INVALID, "layer " + std::to_string(l) + ": a required tensor is null");
        if (L.gate_inp_type != LSTK_TYPE_F16 && L.gate_inp_type != LSTK_TYPE_F32)
            return set_error(LSTK_E_INVALID, "layer " + std::to_string(l) + ": gate_inp must be F16 or F32");
    }

    lstk_model *M = new lstk_model();
    M->hp = hp;
    M->layers.assign(w->layers, w->layers + hp.n_layer);
    M->tok_embd = w->tok_embd;
    M->output = w->output ? w->output : w->tok_embd;
    M->output_norm = w->output_norm;
    M->pool = pool;
    M->streaming = lstk::pool_streaming(pool);
    M->device_lru = lstk::pool_device_lru(pool);
    M->n_batch = (int) n_batch;
    M->theta_scale = powf(hp.rope_freq_base, -2.0f / (float) hp.head_dim);
    M->kv.init(kv_size);

    const size_t nb = n_batch, h = (size_t) hp.n_embd, hq = (size_t) hp.n_head * hp.head_dim,
                 hk = (size_t) hp.n_head_kv * hp.head_dim, k = (size_t) hp.n_expert_used;
    M->layer_elems = (size_t) kv_size * hk;
    const size_t part_rows = lstk::attn_part_rows((int) nb, hp.n_head);
    struct Piece {
        void **dst;
        size_t bytes;
    };
    std::vector<Piece> pieces = {
        {(void **) &M->kcache, 2 * M->layer_elems * hp.n_layer * sizeof(uint16_t)},
        {(void **) &M->x, nb * h * 4},
        {(void **) &M->hn, nb * h * 4},
        {(void **) &M->q, nb * (hq + 2 * hk) * 4},
        {(void **) &M->qr, nb * hq * 2},
        {(void **) &M->attn, nb * hq * 4},
        {(void **) &M->part, part_rows * (hp.head_dim + 4) * 4},
        {(void **) &M->weights, nb * k * 4},
        {(void **) &M->ids, nb * k * 4},
        {(void **) &M->slots, nb * k * 4},
        {(void **) &M->in, 3 * nb * 4},
        {(void **) &M->hn16, nb * h * 2},
        {(void **) &M->attn16, nb * hq * 2},
        {(void **) &M->cell_seq, (size_t) kv_size * 4},
        {(void **) &M->cell_pos, (size_t) kv_size * 4},
        {(void **) &M->rope_cs, nb * (size_t) hp.head_dim * 4},
    };
    size_t total = 0;
    for (const Piece &p : pieces) total += (p.bytes + 255) / 256 * 256;
    hipError_t e = hipMalloc(&M->mem, total);
    if (e != hipSuccess) {
        destroy(M);
        return set_error(LSTK_E_NOMEM, "hipMalloc of " + std::to_string(total) + " bytes failed");
    }
    size_t off = 0;
    for (const Piece &p : pieces) {
        *p.dst = static_cast<uint8_t *>(M->mem) + off;
        off += (p.bytes + 255) / 256 * 256;
    }
    M->vcache = M->kcache + M->layer_elems * hp.n_layer;
    M->ld_qkv = (int) (hq + 2 * hk);
    M->k = M->q + hq;
    M->v = M->k + hk;
    M->qkv_joined.resize(hp.n_layer);
    for (int l = 0; l < hp.n_layer; l++) {
        const lstk_qwen3_layer &L = w->layers[l];
        M->qkv_joined[l] = L.wk == L.wq + hq * h && L.wv == L.wk + hk * h;
    }
    // zero K/V (a masked cell is never read, but keep the cache free of stale NaNs as the reference
    // does, src/kv_cache.cpp:31) and mark every cell empty
    if ((e = hipMemset(M->kcache, 0, 2 * M->layer_elems * hp.n_layer * sizeof(uint16_t))) != hipSuccess ||
        (e = hipMemset(M->cell_seq, 0xff, (size_t) kv_size * 4)) != hipSuccess ||
        (e = hipMemset(M->cell_pos, 0xff, (size_t) kv_size * 4)) != hipSuccess ||
        (e = hipMemset(M->in, 0, (size_t) 3 * nb * 4)) != hipSuccess) {
        destroy(M);
        return hip_fail(e, "hipMemset");
    }
    if ((e = hipHostMalloc((void **) &M->h_in, (3 * nb + 2 * nb * k) * 4, hipHostMallocDefault)) != hipSuccess) {
        destroy(M);
        return set_error(LSTK_E_NOMEM, "hipHostMalloc of the step staging failed");
    }
    if (rocblas_create_handle(&M->blas) != rocblas_status_success) {
        M->blas = nullptr;
        destroy(M);
        return set_error(LSTK_E_DEVICE, "rocblas_create_handle failed");
    }
    M->h_ids = M->h_in + 3 * nb;
    M->h_slots = M->h_ids + nb * k;
    if ((e = hipEventCreateWithFlags(&M->in_free, hipEventDisableTiming)) != hipSuccess ||
        (e = hipEventRecord(M->in_free, nullptr)) != hipSuccess) {
        destroy(M);
        return hip_fail(e, "hipEventCreate");
    }
    *out = M;
    return LSTK_OK;
}

// Records the time of `f`'s work on the stream with events around it (library calls launch kernels of
// their own, which per-launch events cannot see).
template <typename F>
int timed_span(lstk_model *M, int stage, hipStream_t st, F &&f) {
    if (!M->timing) return f();
    TimedLaunch t{};
    if (hipEventCreate(&t.start) != hipSuccess || hipEventCreate(&t.end) != hipSuccess ||
        hipEventRecord(t.start, st) != hipSuccess)
        return set_error(LSTK_E_DEVICE, "timing events");
    const int rc = f();
    if (hipEventRecord(t.end, st) != hipSuccess) return set_error(LSTK_E_DEVICE, "timing events");
    M->launched[stage].push_back(t);
    return rc;
}

// Y[t][r] (+)= sum_c X16[t][c] W[r][c] for T tokens: one rocBLAS f16 x f16 -> f32 product in column-major
// terms, Y^T (rows x T, ld ldy) = W^T-op(A) (rows x cols) . X16^T (cols x T).
int blas_gemm(lstk_model *M, const uint16_t *W, int rows, int cols, const uint16_t *X16, int T, float *Y, int ldy,
              bool accumulate, hipStream_t st) {
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    rocblas_status s = rocblas_set_stream(M->blas, st);
    if (s == rocblas_status_success)
        s = rocblas_gemm_ex(M->blas, rocblas_operation_transpose, rocblas_operation_none, rows, T, cols, &alpha, W,
                            rocblas_datatype_f16_r, cols, X16, rocblas_datatype_f16_r, cols, &beta, Y, rocblas_datatype_f32_r,
                            ldy, Y, rocblas_datatype_f32_r, ldy, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    return s == rocblas_status_success ? LSTK_OK
                                       : set_error(LSTK_E_DEVICE, std::string("rocblas_gemm_ex: ") + rocblas_status_to_string(s));
}

// The same product on the matrix cores for up to 16 tokens (gemm16_kernel), rocBLAS beyond.
int project(lstk_model *M, const uint16_t *W, int rows, int cols, const uint16_t *X16, int T, float *Y, int ldy,
            bool accumulate, hipStream_t st) {
    if (!lstk::gemm16_supported(rows, cols, T)) return blas_gemm(M, W, rows, cols, X16, T, Y, ldy, accumulate, st);
    const lstk::Gemm16Params gp{W, X16, Y, rows, cols, T, ldy, accumulate ? 1 : 0};
    const hipError_t e = lstk::launch_gemm16(gp, st, nullptr);
    return e == hipSuccess ? LSTK_OK : hip_fail(e, "gemm16 launch");
}

// Copies the host bookkeeping of the cells to the device (after removals; rare, synchronous).
int sync_cells(lstk_model *M) {
    hipError_t e;
    if ((e = hipDeviceSynchronize()) != hipSuccess ||
        (e = hipMemcpy(M->cell_seq, M->kv.cell_seq.data(), M->kv.size * 4, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(M->cell_pos, M->kv.cell_pos.data(), M->kv.size * 4, hipMemcpyHostToDevice)) != hipSuccess)
        return hip_fail(e, "cell table upload");
    return LSTK_OK;
}

// The MoE block of layer l on `rows` rows of hn, added into the residual rows xr in place.
// With ffn_norm set (one token, resident pool) the router launch computes hn = rms_norm(xr) * ffn_norm
// itself, so the step needs no RMSNorm launch before the block.
int moe(lstk_model *M, int l, int rows, float *xr, int32_t *ids, hipStream_t st, const float *ffn_norm) {
    const lstk_qwen3_layer &L = M->layers[l];
    if (!M->streaming && ffn_norm)
        return lstk::moe_block_normed(M->pool, l, xr, ffn_norm, M->hp.rms_eps, M->hn, L.gate_inp, L.gate_inp_type, xr, xr,
                                      ids, M->weights, rows, st);
    if (!M->streaming)
        return lstk_moe_block(M->pool, l, M->hn, L.gate_inp, L.gate_inp_type, xr, xr, ids, M->weights, rows, st);
    // Engine::run_segment (src/engine.cpp:343-392): the host sees the router's choice, acquires the
    // experts (misses are copied on the pool's side streams) and the experts run on their slots.
    // With the bookkeeping on the device the same acquire runs as two kernels on `st` instead, and
    // the host never waits.
    const int k = M->hp.n_expert_used;
    int rc = lstk_moe_route(M->pool, l, M->hn, rows, L.gate_inp, L.gate_inp_type, ids, M->weights, st);
    if (rc != LSTK_OK) return rc;
    if (M->device_lru) {
        if ((rc = lstk_pool_acquire_device(M->pool, l, ids, rows * k, M->slots, st)) != LSTK_OK) return rc;
        return lstk_moe_ffn(M->pool, l, M->hn, M->slots, M->weights, xr, xr, rows, st);
    }
    hipError_t e;
    if ((e = hipMemcpyAsync(M->h_ids, ids, (size_t) rows * k * 4, hipMemcpyDeviceToHost, st)) != hipSuccess ||
        (e = hipStreamSynchronize(st)) != hipSuccess)
        return hip_fail(e, "router ids download");
    if ((rc = lstk_pool_acquire(M->pool, l, M->h_ids, rows * k, M->h_slots, st)) != LSTK_OK) {
        (void) lstk_pool_release_all(M->pool, st);
        return rc;
    }
    if ((e = hipMemcpyAsync(M->slots, M->h_slots, (size_t) rows * k * 4, hipMemcpyHostToDevice, st)) != hipSuccess)
        return hip_fail(e, "slot upload");
    rc = lstk_moe_ffn(M->pool, l, M->hn, M->slots, M->weights, xr, xr, rows, st);
    const int rrc = lstk_pool_release_all(M->pool, st);
    return rc != LSTK_OK ? rc : rrc;
}

// Engine::make_step_inputs (src/engine.cpp:200-243): reserves the KV cells of T tokens of seq and queues
// the upload of the tokens, cells and positions to the model's input buffer; *n_cells = the attended cells.
int prepare(lstk_model *M, int32_t seq, const int32_t *tokens, int T, int *n_cells, hipStream_t st) {
    std::vector<int32_t> cells, pos;
    if (!M->kv.alloc(seq, T, cells, pos)) return set_error(LSTK_E_EXHAUSTED, "KV cache is full");
    *n_cells = M->kv.n_kv();
    const int nb = M->n_batch;
    hipError_t e;
    // the staging buffer is reused once the previous step's upload has left it
    if ((e = hipEventSynchronize(M->in_free)) != hipSuccess) return hip_fail(e, "hipEventSynchronize");
    std::memcpy(M->h_in, tokens, (size_t) T * 4);
    std::memcpy(M->h_in + nb, cells.data(), (size_t) T * 4);
    std::memcpy(M->h_in + 2 * nb, pos.data(), (size_t) T * 4);
    if ((e = hipMemcpyAsync(M->in, M->h_in, (size_t) 3 * nb * 4, hipMemcpyHostToDevice, st)) != hipSuccess ||
        (e = hipEventRecord(M->in_free, st)) != hipSuccess)
        return hip_fail(e, "step input upload");
    return LSTK_OK;
}

// The kernels of one step (qwen3_build_graph, src/qwen3.cpp:223-259) over the inputs prepare() uploaded.
// With a resident pool (or a streaming pool that acquires on the device) this makes no host
// synchronisation, so a caller may capture it in a HIP graph.
int forward(lstk_model *M, int32_t seq, int T, int n_cells, float *d_logits, int32_t *d_trace, hipStream_t st) {
    const lstk_qwen3_hparams &hp = M->hp;
    const int nb = M->n_batch, h = hp.n_embd, hd = hp.head_dim, k = hp.n_expert_used;
    const int hq = hp.n_head * hd, hk = hp.n_head_kv * hd;
    hipError_t e;
    const int32_t *d_tok = M->in, *d_cells = M->in + nb, *d_pos = M->in + 2 * nb;
    const bool blas = T >= kBlasMinTokens;
    // The attended range starts at the sequence's lowest block when the step runs now. A captured forward
    // is replayed after later prepares whose new blocks may lie below that block (freed blocks come back
    // in the order they were released), so a capture attends from cell 0: cells of other sequences and
    // free cells are masked, and the cell that holds each new token is always inside the range.
    hipStreamCaptureStatus capturing = hipStreamCaptureStatusNone;
    if ((e = hipStreamIsCapturing(st, &capturing)) != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    const int range_begin =
        capturing == hipStreamCaptureStatusNone ? std::min(M->kv.first_cell(seq), std::max(0, n_cells - 1)) / 64 * 64 : 0;
    {
        // the step's RoPE angles, shared by every layer
        lstk::RopeParams tp{};
        tp.pos = d_pos;
        tp.T = T;
        tp.hd = hd;
        tp.theta_scale = M->theta_scale;
        if ((e = lstk::launch_rope_table(tp, M->rope_cs, st)) != hipSuccess) return hip_fail(e, "rope table launch");
    }

    // A step of several tokens leaves each layer's MoE combine (but the last's) to the next layer's
    // attn_norm launch, which adds the expert rows into the residual and normalises the sum in one
    // launch (the same values as the combine and RMSNorm launches; not when a debug capture wants the
    // residual after each block, nor with a streaming pool).
    const bool defer = T > 1 && !M->streaming && !M->capture && !M->capture_moe;
    bool pending = false; // the previous layer's expert rows wait in the pool's rows
    for (int l = 0; l < hp.n_layer; l++) {
        const lstk_qwen3_layer &L = M->layers[l];
        lstk::GemvParams gp{};
        gp.seg[0] = {L.wq, M->q, nullptr, hq, M->ld_qkv};
        gp.seg[1] = {L.wk, M->k, nullptr, hk, M->ld_qkv};
        gp.seg[2] = {L.wv, M->v, nullptr, hk, M->ld_qkv};
        gp.nseg = 3;
        gp.rows_total = hq + 2 * hk;
        gp.cols = h;
        gp.T = T;
        if (T == 1) {
            // one token: attn_norm (and layer 0's embedding gather) run inside the Q/K/V launch
            gp.x = M->x;
            gp.norm_w = L.attn_norm;
            gp.eps = hp.rms_eps;
            if (l == 0) {
                gp.emb = M->tok_embd;
                gp.tokens = d_tok;
                gp.x_out = M->x;
            }
        } else {
            lstk::NormParams np{M->x, l == 0 ? M->tok_embd : nullptr, d_tok, M->x, L.attn_norm, M->hn, T, h, hp.rms_eps,
                                blas ? M->hn16 : nullptr};
            if (pending) {
                np.Y = lstk::pool_moe_rows(M->pool);
                np.k = k;
                pending = false;
            }
            if ((e = timed(M, 0, [&](const lstk::LaunchTiming *tm) { return lstk::launch_rmsnorm(np, st, tm); })) != hipSuccess)
                return hip_fail(e, "attn_norm launch");
            gp.x = M->hn;
        }
        uint16_t *kc = M->kcache + M->layer_elems * l, *vc = M->vcache + M->layer_elems * l;
        lstk::RopeParams rp{M->q, M->k, M->v, L.q_norm, L.k_norm, hp.rms_eps, d_pos, d_cells, seq, M->cell_seq, M->cell_pos,
                            T, hp.n_head, hp.n_head_kv, hd, (int) M->kv.size, M->theta_scale, M->qr, kc, vc, M->rope_cs,
                            M->ld_qkv};
        // one token (its query rows in one 16-row tile): QK-norm, RoPE and the K / V store run inside
        // the attention launch
        const bool rope_in_attn = T == 1 && hp.n_head / hp.n_head_kv <= 16 && !M->rope_apart;
        if (blas) {
            const int rc = timed_span(M, 1, st, [&] {
                // Q, K and V rows side by side in the output; one product when the weights are too
                if (M->qkv_joined[l]) return project(M, L.wq, hq + 2 * hk, h, M->hn16, T, M->q, M->ld_qkv, false, st);
                int r = project(M, L.wq, hq, h, M->hn16, T, M->q, M->ld_qkv, false, st);
                if (r == LSTK_OK) r = project(M, L.wk, hk, h, M->hn16, T, M->k, M->ld_qkv, false, st);
                if (r == LSTK_OK) r = project(M, L.wv, hk, h, M->hn16, T, M->v, M->ld_qkv, false, st);
                return r;
            });
            if (rc != LSTK_OK) return rc;
        } else if ((e = timed(M, 1, [&](const lstk::LaunchTiming *tm) { return lstk::launch_gemv(gp, st, tm); })) != hipSuccess) {
            return hip_fail(e, "qkv launch");
        }
        lstk::AttnParams ap{};
        ap.q = M->qr;
        ap.kc = kc;
        ap.vc = vc;
        ap.cell_seq = M->cell_seq;
        ap.cell_pos = M->cell_pos;
        ap.pos = d_pos;
        ap.seq = seq;
        ap.T = T;
        ap.n_head = hp.n_head;
        ap.n_kv = hp.n_head_kv;
        ap.hd = hd;
        ap.kv_size = (int) M->kv.size;
        ap.n_cells = n_cells;
        ap.cell_begin = range_begin;
        ap.scale = 1.0f / sqrtf((float) hd);
        ap.part = M->part;
        ap.out = M->attn;
        ap.out16 = blas ? M->attn16 : nullptr;
        ap.rope_in = rope_in_attn ? 1 : 0;
        ap.rope = rp;
        lstk::attn_plan(ap); // clears rope_in when the context is too long for one pass per chunk
        if (!ap.rope_in && (e = timed(M, 1, [&](const lstk::LaunchTiming *tm) { return lstk::launch_rope(rp, st, tm); })) != hipSuccess)
            return hip_fail(e, "rope launch");
        if ((e = timed(M, 2, [&](const lstk::LaunchTiming *tm) { return lstk::launch_attn(ap, st, tm); })) != hipSuccess ||
            (ap.n_chunk > 1 &&
             (e = timed(M, 2, [&](const lstk::LaunchTiming *tm) { return lstk::launch_attn_combine(ap, st, tm); })) != hipSuccess))
            return hip_fail(e, "attention launch");
        lstk::GemvParams op{};
        op.seg[0] = {L.wo, M->x, M->x, h, h};
        op.nseg = 1;
        op.rows_total = h;
        op.cols = hq;
        op.x = M->attn;
        op.T = T;
        // after the last attention only the output row goes on (src/qwen3.cpp:233-237)
        const bool last = l == hp.n_layer - 1;
        const int rows = last ? 1 : T;
        float *xr = M->x + (size_t) (T - rows) * h;
        lstk::NormParams fp{xr, nullptr, nullptr, nullptr, L.ffn_norm, M->hn, rows, h, hp.rms_eps};
        if (blas) {
            const int rc = timed_span(M, 3, st, [&] { return project(M, L.wo, h, hq, M->attn16, T, M->x, h, true, st); });
            if (rc != LSTK_OK) return rc;
        } else if ((e = timed(M, 3, [&](const lstk::LaunchTiming *tm) { return lstk::launch_gemv(op, st, tm); })) != hipSuccess) {
            return hip_fail(e, "o-proj launch");
        }
        if (M->capture_moe && (e = hipMemcpyAsync(M->capture_moe + (size_t) l * T * h, M->x, (size_t) T * h * sizeof(float),
                                                  hipMemcpyDeviceToDevice, st)) != hipSuccess)
            return hip_fail(e, "capture copy");
        // ffn_norm inside the router launch (resident pools) up to 63 rows: a 512-token prompt measured 1.6%
        // slower that way (each row normalised by every expert group's work-group) than with its own launch
        const bool norm_in_router = !M->streaming && rows < 64;
        if (!norm_in_router &&
            (e = timed(M, 0, [&](const lstk::LaunchTiming *tm) { return lstk::launch_rmsnorm(fp, st, tm); })) != hipSuccess)
            return hip_fail(e, "ffn_norm launch");
        int32_t *ids = d_trace ? d_trace + ((size_t) l * T + (T - rows)) * k : M->ids;
        if (last && d_trace && T > 1) {
            lstk::FillParams fl{d_trace + (size_t) l * T * k, (T - 1) * k, -1};
            if ((e = lstk::launch_fill(fl, st, nullptr)) != hipSuccess) return hip_fail(e, "trace fill launch");
        }
        const bool defer_here = defer && !last;
        if (defer_here) lstk::pool_defer_combine(M->pool, true);
        const int rc = moe(M, l, rows, xr, ids, st, norm_in_router ? L.ffn_norm : nullptr);
        if (defer_here) lstk::pool_defer_combine(M->pool, false);
        if (rc != LSTK_OK) return rc;
        pending = defer_here;
        if (M->capture && (e = hipMemcpyAsync(M->capture + (size_t) l * T * h, M->x, (size_t) T * h * sizeof(float),
                                              hipMemcpyDeviceToDevice, st)) != hipSuccess)
            return hip_fail(e, "capture copy");
    }
    lstk::NormParams onp{M->x + (size_t) (T - 1) * h, nullptr, nullptr, nullptr, M->output_norm, M->hn, 1, h, hp.rms_eps};
    if ((e = timed(M, 0, [&](const lstk::LaunchTiming *tm) { return lstk::launch_rmsnorm(onp, st, tm); })) != hipSuccess)
        return hip_fail(e, "output_norm launch");
    lstk::GemvParams hpp{};
    hpp.seg[0] = {M->output, d_logits, nullptr, hp.n_vocab, hp.n_vocab};
    hpp.nseg = 1;
    hpp.rows_total = hp.n_vocab;
    hpp.cols = h;
    hpp.x = M->hn;
    hpp.T = 1;
    if ((e = timed(M, 4, [&](const lstk::LaunchTiming *tm) { return lstk::launch_gemv(hpp, st, tm); })) != hipSuccess)
        return hip_fail(e, "output head launch");
    return LSTK_OK;
}

int step(lstk_model *M, int32_t seq, const int32_t *tokens, int T, float *d_logits, int32_t *d_trace, hipStream_t st) {
    int n_cells = 0;
    const int rc = prepare(M, seq, tokens, T, &n_cells, st);
    return rc != LSTK_OK ? rc : forward(M, seq, T, n_cells, d_logits, d_trace, st);
}

int check_tokens(const lstk_model *M, const int32_t *tokens, int n) {
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= M->hp.n_vocab)
            return set_error(LSTK_E_INVALID, "token id " + std::to_string(tokens[i]) + " out of range");
    return LSTK_OK;
}

}  // namespace

extern "C" {

int lstk_model_create(const lstk_qwen3_hparams *hp, const lstk_qwen3_weights *w, lstk_pool *pool, uint32_t kv_size,
                      uint32_t n_batch, lstk_model **out) {
    try {
        return create(hp, w, pool, kv_size, n_batch, out);
    } catch (const std::exception &ex) {
        return set_error(LSTK_E_NOMEM, std::string("lstk_model_create: ") + ex.what());
    }
}

void lstk_model_destroy(lstk_model *model) { destroy(model); }

int lstk_model_decode(lstk_model *model, int32_t seq, const int32_t *tokens, int n_tokens, float *d_logits,
                      int32_t *d_trace, lstk_stream_t stream) {
    if (!model) return set_error(LSTK_E_INVALID, "null model");
    if (n_tokens < 1 || !tokens || !d_logits) return set_error(LSTK_E_INVALID, "need at least one token and a logits buffer");
    if (seq < 0) return set_error(LSTK_E_INVALID, "seq must be >= 0");
    if (check_tokens(model, tokens, n_tokens) != LSTK_OK) return LSTK_E_INVALID;
    hipStream_t st = static_cast<hipStream_t>(stream);
    try {
        for (int done = 0; done < n_tokens;) {
            const int n = std::min(model->n_batch, n_tokens - done);
            int32_t *tr = d_trace ? d_trace : model->trace ? model->trace_dev : nullptr;
            const int rc = step(model, seq, tokens + done, n, d_logits, tr, st);
            if (rc != LSTK_OK) return rc;
            if (model->trace) {
                // Engine::step_resident's trace write (src/engine.cpp:299-316): token count, then each layer's ids
                const size_t cnt = (size_t) model->hp.n_layer * n * model->hp.n_expert_used;
                model->trace_host.resize(cnt);
                hipError_t e;
                if ((e = hipMemcpyAsync(model->trace_host.data(), tr, cnt * 4, hipMemcpyDeviceToHost, st)) != hipSuccess ||
                    (e = hipStreamSynchronize(st)) != hipSuccess)
                    return hip_fail(e, "trace download");
                const int32_t n32 = n;
                if (fwrite(&n32, 4, 1, model->trace) != 1 || fwrite(model->trace_host.data(), 4, cnt, model->trace) != cnt ||
                    fflush(model->trace) != 0)
                    return set_error(LSTK_E_IO, "routing trace write failed");
            }
            done += n;
        }
    } catch (const std::exception &ex) {
        return set_error(LSTK_E_NOMEM, std::string("lstk_model_decode: ") + ex.what());
    }
    return LSTK_OK;
}

int lstk_model_prepare(lstk_model *model, int32_t seq, const int32_t *tokens, int n_tokens, int32_t *n_cells,
                       lstk_stream_t stream) {
    if (!model || !tokens || !n_cells) return set_error(LSTK_E_INVALID, "null argument");
    if (seq < 0 || n_tokens < 1 || n_tokens > model->n_batch)
        return set_error(LSTK_E_INVALID, "seq must be >= 0 and n_tokens in [1, n_batch]");
    if (check_tokens(model, tokens, n_tokens) != LSTK_OK) return LSTK_E_INVALID;
    try {
        int nc = 0;
        const int rc = prepare(model, seq, tokens, n_tokens, &nc, static_cast<hipStream_t>(stream));
        *n_cells = nc;
        return rc;
    } catch (const std::exception &ex) {
        return set_error(LSTK_E_NOMEM, std::string("lstk_model_prepare: ") + ex.what());
    }
}

int lstk_model_forward(lstk_model *model, int32_t seq, int n_tokens, int32_t n_cells, float *d_logits, int32_t *d_trace,
                       lstk_stream_t stream) {
    if (!model || !d_logits) return set_error(LSTK_E_INVALID, "null argument");
    if (seq < 0 || n_tokens < 1 || n_tokens > model->n_batch || n_cells < 1 || n_cells > (int32_t) model->kv.size)
        return set_error(LSTK_E_INVALID, "seq must be >= 0, n_tokens in [1, n_batch], n_cells in [1, kv_size]");
    return forward(model, seq, n_tokens, n_cells, d_logits, d_trace, static_cast<hipStream_t>(stream));
}

int lstk_model_fill_context(lstk_model *model, int32_t seq, int n_cells, uint64_t seed, lstk_stream_t stream) {
    if (!model) return set_error(LSTK_E_INVALID, "null model");
    if (seq < 0 || n_cells < 0) return set_error(LSTK_E_INVALID, "seq and n_cells must be >= 0");
    lstk_model *M = model;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int nb = M->n_batch;
    try {
        for (int done = 0; done < n_cells;) {
            const int T = std::min(nb, n_cells - done);
            std::vector<int32_t> cells, pos;
            if (!M->kv.alloc(seq, T, cells, pos)) return set_error(LSTK_E_EXHAUSTED, "KV cache is full");
            hipError_t e;
            if ((e = hipEventSynchronize(M->in_free)) != hipSuccess) return hip_fail(e, "hipEventSynchronize");
            std::memcpy(M->h_in + nb, cells.data(), (size_t) T * 4);
            std::memcpy(M->h_in + 2 * nb, pos.data(), (size_t) T * 4);
            if ((e = hipMemcpyAsync(M->in, M->h_in, (size_t) 3 * nb * 4, hipMemcpyHostToDevice, st)) != hipSuccess ||
                (e = hipEventRecord(M->in_free, st)) != hipSuccess)
                return hip_fail(e, "context upload");
            lstk::FillKvParams fp{M->in + nb, M->in + 2 * nb, seq, M->cell_seq, M->cell_pos, T, M->hp.n_layer,
                                  M->hp.n_head_kv, M->hp.head_dim, (int) M->kv.size, M->layer_elems, M->kcache,
                                  M->vcache, seed};
            if ((e = lstk::launch_fill_kv(fp, st, nullptr)) != hipSuccess) return hip_fail(e, "fill launch");
            done += T;
        }
    } catch (const std::exception &ex) {
        return set_error(LSTK_E_NOMEM, std::string("lstk_model_fill_context: ") + ex.what());
    }
    return LSTK_OK;
}

int lstk_model_debug_capture(lstk_model *model, float *d_states) {
    if (!model) return set_error(LSTK_E_INVALID, "null model");
    model->capture = d_states;
    return LSTK_OK;
}

int lstk_model_debug_capture_moe_in(lstk_model *model, float *d_moe_in) {
    if (!model) return set_error(LSTK_E_INVALID, "null model");
    model->capture_moe = d_moe_in;
    return LSTK_OK;
}

int lstk_model_set_trace(lstk_model *model, const char *path) {
    if (!model) return set_error(LSTK_E_INVALID, "null model");
    if (model->trace) {
        fclose(model->trace);
        model->trace = nullptr;
    }
    if (!path) return LSTK_OK;
    if (!model->trace_dev) {
        const size_t bytes = (size_t) model->hp.n_layer * model->n_batch * model->hp.n_expert_used * 4;
        const hipError_t e = hipMalloc(&model->trace_dev, bytes);
        if (e != hipSuccess) {
            model->trace_dev = nullptr;
            return set_error(LSTK_E_NOMEM, "hipMalloc of the trace buffer failed");
        }
    }
    model->trace = fopen(path, "wb");
    if (!model->trace) return set_error(LSTK_E_IO, std::string("cannot write ") + path);
    static const char magic[8] = {'L', 'S', 'T', 'K', 'R', 'T', 'E', '1'};
    const int32_t header[3] = {model->hp.n_layer, model->hp.n_expert, model->hp.n_expert_used};
    if (fwrite(magic, 1, 8, model->trace) != 8 || fwrite(header, 4, 3, model->trace) != 3 || fflush(model->trace) != 0)
        return set_error(LSTK_E_IO, "routing trace write failed");
    return LSTK_OK;
}

int lstk_model_remove_seq(lstk_model *model, int32_t seq) {
    if (!model) return set_error(LSTK_E_INVALID, "null model");
    model->kv.remove_seq(seq);
    return sync_cells(model);
}

int lstk_model_truncate_seq(lstk_model *model, int32_t seq, int32_t keep) {
    if (!model) return set_error(LSTK_E_INVALID, "null model");
    model->kv.truncate_seq(seq, keep);
    return sync_cells(model);
}

int32_t lstk_model_seq_len(const lstk_model *model, int32_t seq) {
    if (!model) return 0;
    return model->kv.length(seq);
}

int lstk_model_debug_options(lstk_model *model, int flags) {
    if (!model) return set_error(LSTK_E_INVALID, "null model");
    if (flags & ~1) return set_error(LSTK_E_INVALID, "unknown debug option bits");
    model->rope_apart = (flags & 1) != 0;
    return LSTK_OK;
}

int lstk_debug_attn_plan(int n_tokens, int n_head, int n_kv, int head_dim, int kv_size, int n_cells, int cell_begin,
                         int rope_in, int32_t out[6]) {
    if (!out || n_tokens < 1 || n_head < 1 || n_kv < 1 || n_head % n_kv || !lstk::attn_supported(head_dim) ||
        kv_size < 32 || kv_size % 32 || n_cells < 1 || n_cells > kv_size || cell_begin < 0 || cell_begin >= n_cells ||
        cell_begin % 64)
        return set_error(LSTK_E_INVALID, "lstk_debug_attn_plan: bad arguments");
    lstk::AttnParams ap{};
    ap.T = n_tokens;
    ap.n_head = n_head;
    ap.n_kv = n_kv;
    ap.hd = head_dim;
    ap.kv_size = kv_size;
    ap.n_cells = n_cells;
    ap.cell_begin = cell_begin;
    ap.rope_in = rope_in ? 1 : 0;
    lstk::attn_plan(ap);
    out[0] = ap.rb_rows;
    out[1] = ap.n_rowblk;
    out[2] = ap.chunk;
    out[3] = ap.n_chunk;
    out[4] = ap.rope_in;
    out[5] = n_kv * ap.n_chunk * ap.n_rowblk;
    return LSTK_OK;
}

int lstk_model_set_timing(lstk_model *model, int enable) {
    if (!model) return set_error(LSTK_E_INVALID, "null model");
    model->timing = enable != 0;
    return LSTK_OK;
}

int lstk_model_timing(lstk_model *model, double ms[5], int64_t launches[5]) {
    if (!model || !ms || !launches) return set_error(LSTK_E_INVALID, "null argument");
    for (int s = 0; s < kStages; s++) {
        ms[s] = 0.0;
        launches[s] = 0;
        for (TimedLaunch &t : model->launched[s]) {
            hipError_t e = hipEventSynchronize(t.end);
            if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
            float v = 0.0f;
            if ((e = hipEventElapsedTime(&v, t.start, t.end)) != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
            ms[s] += v;
            launches[s]++;
            (void) hipEventDestroy(t.start);
            (void) hipEventDestroy(t.end);
        }
        model->launched[s].clear();
    }
    return LSTK_OK;
}

}  // extern "C"
