// qmm_api.hip — the C ABI declared in include/qmm_hip.h: context, device
// memory, argument validation and the multi-task dispatcher.
//
// The dispatcher mirrors sdot_gemm_multi_dispatch (E:4188-4262): tasks are
// laid out in one concatenated row space (start_row, E:4196-4197), the
// activations are quantized once per call into the context's buffers
// (Q8_K when any K-quant task is present, Q8_0 when any Q8_0 task is,
// E:4198-4215), and every task runs on the shared quantized input. Where the
// reference splits the row space over a spinning CPU pool (E:3491-3619),
// each task here is one kernel launch on the context's stream: M = 1 goes to
// the GEMV kernels, M >= 2 to the MFMA kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/qmm_hip.h"
#include "qmm_device.h"

// Device scratch of qmm_gemm_multi_dispatch_noalloc: the quantized input
// of one call (its Q8_K section, then its Q8_0 section). Every GPU the
// library runs on holds its own copy until the process ends. In host code
// `scratch` names a host-side stand-in, never device memory: kernels and
// copies get the device address that hipGetSymbolAddress returns for the
// current device (scratch_on, filled at qmm_init).
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_on[kMaxDevices] = {};  // the array's address on each device, once looked up
}  // namespace

struct qmm_context {
    int device = 0;
    void *scratch = nullptr;  // this device's copy of `scratch` (nullptr: lookup failed)
    std::string scratch_err;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    void *act = nullptr;  // Q8_K + Q8_0 activation buffers of the dispatcher
    size_t act_cap = 0;
    void *lm = nullptr;   // LM-head epilogue scratch: logits | argmax slices | gathered rows
    size_t lm_cap = 0;
    qmm::ScanFold *fold = nullptr;  // the one-launch scan's state (cleared once, then by every scan's last step)
    bool capturing = false;
    // Instantiated graphs still alive (qmm_graph_end .. qmm_graph_destroy):
    // while any is, a buffer that must grow is replaced but not freed — the
    // graphs keep reading and writing the old one — and is freed once the
    // last of them is destroyed.
    int live_graphs = 0;
    std::vector<void *> retired;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::string err;
};

namespace {

int fail(qmm_context *ctx, int code, const std::string &msg) {
    if (ctx) ctx->err = msg;
    return code;
}

int hip_fail(qmm_context *ctx, hipError_t e, const char *what) {
    return fail(ctx, QMM_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Make ctx->device current for the calling thread.
int use_device(qmm_context *ctx) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGetDevice");
    if (cur != ctx->device) {
        e = hipSetDevice(ctx->device);
        if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
    }
    return QMM_OK;
}

bool supported(uint32_t t) {
    return t == qmm::kF32 || t == qmm::kF16 || t == qmm::kQ8_0 || t == qmm::kQ4_K || t == qmm::kQ5_K ||
           t == qmm::kQ6_K;
}
bool is_float(uint32_t t) { return t == qmm::kF32 || t == qmm::kF16; }
// values per block; F32 / F16 rows are read in 16-B pieces of 8 fp16 / 4
// fp32 values and 32-value MFMA steps, so their K must be a multiple of 32
int block_values(uint32_t t) { return t == qmm::kQ8_0 ? 32 : is_float(t) ? 32 : 256; }

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Grow one of the context's device buffers to `bytes`. During a capture
// nothing may be allocated; while instantiated graphs hold the old buffer it
// is retired (kept) instead of freed.
int grow(qmm_context *ctx, void *&buf, size_t &cap, size_t bytes, const char *what) {
    if (bytes <= cap) return QMM_OK;
    if (ctx->capturing)
        return fail(ctx, QMM_ENOMEM, std::string(what) +
                                         " too small during graph capture: size it before capturing (qmm_reserve)");
    if (buf) {
        if (ctx->live_graphs > 0) {
            ctx->retired.push_back(buf);
        } else {
            (void)hipStreamSynchronize(ctx->stream);
            hipError_t e = hipFree(buf);
            if (e != hipSuccess) {
                buf = nullptr;
                cap = 0;
                return hip_fail(ctx, e, "hipFree");
            }
        }
        buf = nullptr;
        cap = 0;
    }
    hipError_t e = hipMalloc(&buf, bytes);
    if (e != hipSuccess) {
        buf = nullptr;
        (void)hipGetLastError();
        return fail(ctx, QMM_ENOMEM, std::string("hipMalloc of ") + what + " failed");
    }
    cap = bytes;
    return QMM_OK;
}

int ensure_act(qmm_context *ctx, size_t bytes) {
    return grow(ctx, ctx->act, ctx->act_cap, bytes, "activation buffers");
}

int ensure_lm(qmm_context *ctx, size_t bytes) { return grow(ctx, ctx->lm, ctx->lm_cap, bytes, "LM-head scratch"); }

// the one-launch scan's state: allocated once (outside a capture) and
// cleared by a kernel on the context's stream; false where it cannot be
// (the caller then takes the per-chunk launches)
bool ensure_fold(qmm_context *ctx) {
    if (ctx->fold) return true;
    if (ctx->capturing) return false;
    void *p = nullptr;
    if (hipMalloc(&p, sizeof(qmm::ScanFold)) != hipSuccess) return false;
    if (qmm::launch_scan_fold_clear(static_cast<qmm::ScanFold *>(p), ctx->stream) != hipSuccess) {
        (void)hipFree(p);
        return false;
    }
    ctx->fold = static_cast<qmm::ScanFold *>(p);
    return true;
}

void free_retired(qmm_context *ctx) {
    if (ctx->retired.empty()) return;
    (void)hipStreamSynchronize(ctx->stream);
    for (void *p : ctx->retired) (void)hipFree(p);
    ctx->retired.clear();
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// The FFN block's scratch for N intermediate values: h's Q8_K (separate
// launches) or h in fp16 (one launch), then h itself when the caller does not
// take it.
size_t ffn_scratch_bytes(int N) { return align256(qmm::Q8KLayout(1, N).total) + align256(size_t(N) * 4); }

// Validate the task list against (M, K) and assign start_row.
// need_q8k: a K-quant task, or an F32 / F16 task (they read the fp16
// section of the Q8_K buffer when M >= 2 or the input is prequantized)
int check_tasks(qmm_context *ctx, int M, int K, qmm_matrix_task *tasks, int n_tasks,
                bool *need_q8k, bool *need_q80) {
    if (M <= 0 || K <= 0) return fail(ctx, QMM_EINVAL, "M and K must be positive");
    if (!tasks || n_tasks <= 0) return fail(ctx, QMM_EINVAL, "empty task list");
    if (n_tasks > 256) return fail(ctx, QMM_EINVAL, "more than 256 tasks in one dispatch");
    // the M >= 2 kernels address the activation codes with 32-bit offsets
    if (M > 1 && int64_t(M) * int64_t(K) >= (int64_t(1) << 31))
        return fail(ctx, QMM_ESHAPE, "M * K must stay below 2^31 for M >= 2");
    *need_q8k = *need_q80 = false;
    int total = 0;
    for (int t = 0; t < n_tasks; ++t) {
        qmm_matrix_task &T = tasks[t];
        if (!supported(T.type)) return fail(ctx, QMM_ETYPE, "task " + std::to_string(t) + ": unsupported ggml type " + std::to_string(T.type));
        if (T.rows < 0) return fail(ctx, QMM_EINVAL, "task " + std::to_string(t) + ": negative rows");
        if (T.cols != K) return fail(ctx, QMM_ESHAPE, "task " + std::to_string(t) + ": cols != K");
        if (K % block_values(T.type)) return fail(ctx, QMM_ESHAPE, "task " + std::to_string(t) + ": K not a multiple of the block size");
        if (T.row_bytes != qmm_row_bytes(T.type, K)) return fail(ctx, QMM_ESHAPE, "task " + std::to_string(t) + ": row_bytes does not match the type");
        if (T.rows > 0) {
            if (!T.w_base || !T.dst) return fail(ctx, QMM_EINVAL, "task " + std::to_string(t) + ": null weight or dst");
            if (M > 1 && T.dst_stride < size_t(T.rows)) return fail(ctx, QMM_EINVAL, "task " + std::to_string(t) + ": dst_stride < rows");
            if (T.residual && M > 1 && T.res_stride < size_t(T.rows)) return fail(ctx, QMM_EINVAL, "task " + std::to_string(t) + ": res_stride < rows");
            const uintptr_t wa = (T.type == qmm::kQ4_K || T.type == qmm::kQ5_K || is_float(T.type)) ? 16 : 2;
            if (!aligned(T.w_base, wa)) return fail(ctx, QMM_EALIGN, "task " + std::to_string(t) + ": weight base misaligned for its format");
            if (!aligned(T.dst, 4) || (T.residual && !aligned(T.residual, 4))) return fail(ctx, QMM_EALIGN, "task " + std::to_string(t) + ": dst/residual not 4-B aligned");
        }
        if (M == 1 && qmm::gemv_mixed_lds_bytes(T.type, K) > 65536)
            return fail(ctx, QMM_ESHAPE, "task " + std::to_string(t) + ": K too large for the batch-1 kernel");
        if (T.type == qmm::kQ8_0) *need_q80 = true;
        else *need_q8k = true;
        T.start_row = total;  // E:4196-4197
        total += T.rows;
    }
    return QMM_OK;
}

// Kernel views of prequantized activation buffers (a null buffer gives a
// null view).
void act_views(const void *q8k, const void *q80, int M, int K, qmm::Q8KView &xk, qmm::Q80View &x0) {
    xk = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    x0 = {nullptr, nullptr};
    if (q8k) {
        const qmm::Q8KLayout L(M, K);
        const uint8_t *b = static_cast<const uint8_t *>(q8k);
        xk = {reinterpret_cast<const int8_t *>(b), reinterpret_cast<const float *>(b + L.d_off),
              reinterpret_cast<const int32_t *>(b + L.bs_off), reinterpret_cast<const int8_t *>(b + L.tile_off),
              reinterpret_cast<const uint16_t *>(b + L.h_off), reinterpret_cast<const uint16_t *>(b + L.bh_off)};
    }
    if (q80) {
        const qmm::Q80Layout L(M, K);
        const uint8_t *b = static_cast<const uint8_t *>(q80);
        x0 = {reinterpret_cast<const int8_t *>(b), reinterpret_cast<const float *>(b + L.d_off)};
    }
}

qmm::MatArgs mat_args(const qmm_matrix_task &T, int M, int K, const int32_t *scan = nullptr) {
    qmm::MatArgs a;
    a.w = static_cast<const uint8_t *>(T.w_base);
    a.type = T.type;
    a.row_bytes = T.row_bytes;
    a.N = T.rows;
    a.K = K;
    a.M = M;
    a.y = T.dst;
    a.ldy = M > 1 ? T.dst_stride : size_t(T.rows);
    a.res = T.residual;
    a.ldr = M > 1 ? T.res_stride : size_t(T.rows);
    a.scan = scan;
    return a;
}

// x32 != nullptr (M = 1 only): the GEMV kernels quantize x themselves.
// Launches: tasks of one type go together (up to kMaxGroup per launch, in
// order of first appearance); a group of several types — the engine's
// {qkv, gate, alpha, beta} and {q, k, v} groups (E:7954-7959, E:8110-8114) —
// runs as one launch whose workgroups each take their own task's format,
// where that launch applies (M = 1 always; 2 <= M <= 64 with K <= 3072 and
// no Q8_0 task). Outputs are disjoint, so grouping changes no result.
int run_tasks(qmm_context *ctx, const float *x32, const void *q8k, const void *q80, int M, int K,
              const qmm_matrix_task *tasks, int n_tasks, const int32_t *scan = nullptr) {
    qmm::Q8KView xk;
    qmm::Q80View x0;
    act_views(q8k, q80, M, K, xk, x0);
    int nlive = 0;
    bool mixed = false;
    for (int t = 0; t < n_tasks; ++t) {
        if (tasks[t].rows == 0) continue;
        ++nlive;
        for (int u = 0; u < t; ++u)
            if (tasks[u].rows > 0 && tasks[u].type != tasks[t].type) mixed = true;
    }
    if (mixed && nlive <= qmm::kMaxGroup) {
        qmm::MatArgs group[qmm::kMaxGroup];
        int n = 0;
        for (int t = 0; t < n_tasks; ++t)
            if (tasks[t].rows > 0) group[n++] = mat_args(tasks[t], M, K, scan);
        const hipError_t e = (M == 1) ? qmm::launch_gemv_mixed(group, n, x32, xk, x0, ctx->stream)
                                      : qmm::launch_mfma_mixed(group, n, xk, ctx->stream);
        if (e == hipSuccess) return QMM_OK;
        if (e != hipErrorNotSupported) return hip_fail(ctx, e, "matmul launch");
    }
    bool done[256] = {};
    for (int t0 = 0; t0 < n_tasks; ++t0) {
        if (done[t0] || tasks[t0].rows == 0) continue;
        qmm::MatArgs group[qmm::kMaxGroup];
        int n = 0;
        for (int t = t0; t < n_tasks; ++t) {
            const qmm_matrix_task &T = tasks[t];
            if (done[t] || T.rows == 0 || T.type != tasks[t0].type) continue;
            done[t] = true;
            group[n++] = mat_args(T, M, K, scan);
            if (n == qmm::kMaxGroup) break;
        }
        const hipError_t e = (M == 1) ? qmm::launch_gemv(tasks[t0].type, group, n, x32, xk, x0, ctx->stream)
                                      : qmm::launch_mfma(tasks[t0].type, group, n, xk, x0, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "matmul launch");
    }
    return QMM_OK;
}

// Checks of a prequantized input for a validated task list.
// Sections of the dispatcher's own Q8_K buffer that no kernel of an M >= 2
// call reads: bsum32 (read only by the batch-1 GEMV on prequantized input;
// its 2..4-token form sums the codes itself), the row-major codes above 64
// tokens (the tile and slab kernels read the tiles section), the fp16 values
// without an F32 / F16 task.
unsigned q8k_skip(int M, const qmm_matrix_task *tasks, int n_tasks) {
    unsigned skip = qmm::kSkipBs;
    if (M > 64) skip |= qmm::kSkipQs;
    bool flt = false;
    for (int i = 0; i < n_tasks; ++i) flt = flt || is_float(tasks[i].type);
    if (!flt) skip |= qmm::kSkipH;
    return skip;
}

int check_pre(qmm_context *ctx, const void *q8k, const void *q80, bool need_q8k, bool need_q80) {
    if (need_q8k && !q8k) return fail(ctx, QMM_EINVAL, "K-quant or F32/F16 task without Q8_K activations");
    if (need_q80 && !q80) return fail(ctx, QMM_EINVAL, "Q8_0 task without Q8_0 activations");
    if ((q8k && !aligned(q8k, 16)) || (q80 && !aligned(q80, 16)))
        return fail(ctx, QMM_EALIGN, "activation buffers must be 16-B aligned");
    return QMM_OK;
}

// LM-head scratch of one call: logits (unless the caller takes them) |
// argmax partials (per 1024-row slice, or at M = 1 per workgroup of the
// fused grid) | gathered rows (indexed form)
struct LmScratch {
    size_t logit_b, part_b, gather_b;
    size_t total() const { return logit_b + part_b + gather_b; }
};
LmScratch lm_scratch(int M, int rows, size_t row_bytes, bool own_logits, bool gathered) {
    LmScratch L;
    L.logit_b = own_logits ? 0 : align256(size_t(M) * rows * 4);
    L.part_b = align256(std::max(qmm::argmax_scratch_bytes(M, rows),
                                 M == 1 ? size_t(qmm::kMaxArgmaxParts) * sizeof(qmm::Best) : size_t(0)));
    L.gather_b = gathered ? align256(size_t(rows) * row_bytes) : 0;
    return L;
}

// The task of `rows` rows of one tensor (contiguous from w, or gathered by
// id) on M prequantized activation rows, validated before anything is
// launched.
int lm_task(qmm_context *ctx, const void *q8k, const void *q80, int M, int K, const void *w, uint32_t type, int rows,
            float *dst, qmm_matrix_task &t) {
    if (!w || M <= 0 || K <= 0 || rows <= 0) return fail(ctx, QMM_EINVAL, "bad LM-head arguments");
    if (!supported(type)) return fail(ctx, QMM_ETYPE, "unsupported ggml type");
    t = qmm_matrix_task{};
    t.w_base = w;
    t.type = type;
    t.row_bytes = qmm_row_bytes(type, K);
    t.dst = dst ? dst : reinterpret_cast<float *>(uintptr_t(256));  // (placeholder until the scratch exists)
    t.dst_stride = size_t(rows);
    t.rows = rows;
    t.cols = K;
    bool need_q8k, need_q80;
    int rc = check_tasks(ctx, M, K, &t, 1, &need_q8k, &need_q80);
    if (rc) return rc;
    return check_pre(ctx, q8k, q80, need_q8k, need_q80);
}

// One chunk or row list through the LM-head epilogue into (best_val,
// best_id): ids != NULL gathers rows ids[0..rows) of the tensor at w (ids at
// or past id_limit are never read and count as -1e30, E:11150); else rows
// [row_base, row_base + rows) start at w. scr: this call's scratch (laid out
// by lm_scratch); scan: a scan's state or NULL. Arguments are validated.
// A batch-1 scan chunk's step not yet applied: the next chunk's launch
// applies it first (PrevStep), or one scan_final launch does. Its partials
// and the next chunk's alternate between two buffers.
struct PendingStep {
    bool on = false;
    const void *part = nullptr;
    int nparts = 0;
    uint32_t row_base = 0;
    float thresh = 0.0f;
    bool checkpoint = false;
    int c = 0;
    void *bufs[2] = {nullptr, nullptr};
    int launches = 0;  // the scan's launches so far: consecutive ones alternate buffers
    bool seed = false;  // the next launch is the scan's first and seeds its state (no init launch)
    const float *x32 = nullptr;    // non-null: every chunk launch takes this row before its RMSNorm
    const float *gamma = nullptr;  // (the norm's weights)
};

int launch_pending(qmm_context *ctx, PendingStep &pend, float *best_val, uint32_t *best_id, const qmm::ScanStep &st,
                   int32_t *scan) {
    if (!pend.on) return QMM_OK;
    pend.on = false;
    const hipError_t e = qmm::launch_scan_final(pend.part, pend.nparts, pend.row_base, best_val, best_id, st.cand,
                                                st.draft, st.margin, pend.thresh, pend.checkpoint, pend.c, scan,
                                                ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "scan step launch");
}

int lm_argmax_run(qmm_context *ctx, const void *q8k, const void *q80, int M, int K, qmm_matrix_task t,
                  uint32_t row_base, const uint32_t *ids, uint32_t id_limit, float *logits_out, float *best_val,
                  uint32_t *best_id, uint8_t *scr, int32_t *scan, const qmm::ScanStep *step,
                  PendingStep *pend = nullptr) {
    const int rows = t.rows;
    const LmScratch L = lm_scratch(M, rows, t.row_bytes, logits_out != nullptr, ids != nullptr);
    float *logits = logits_out ? logits_out : reinterpret_cast<float *>(scr);
    void *part = scr + L.logit_b;
    hipError_t e;
    if (ids) {
        uint8_t *g = scr + L.logit_b + L.part_b;
        e = qmm::launch_gather_rows(static_cast<const uint8_t *>(t.w_base), t.row_bytes, ids, id_limit, rows, g, scan,
                                    ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "row gather launch");
        t.w_base = g;
    }
    t.dst = logits;
    qmm::Q8KView xk;
    qmm::Q80View x0;
    act_views(q8k, q80, M, K, xk, x0);
    const bool round16 = ids == nullptr;  // chunk scans compare fp16 logits (E:11175), indexed rows fp32
    if (M == 1 && step && pend) {  // a scan chunk: its step waits for the next chunk's launch
        void *mine = pend->bufs[pend->launches++ & 1];
        qmm::PrevStep pre{};
        if (pend->on)
            pre = qmm::PrevStep{pend->part, pend->nparts, pend->row_base, pend->thresh, pend->checkpoint ? 1 : 0,
                                pend->c, best_val, best_id, scan};
        const bool seed = pend->seed;  // (then the state is not read: it is this launch's to write)
        if (seed) {
            pre.best_val = best_val;
            pre.best_id = best_id;
            pre.st = scan;
            pre.init = 1;
            pend->seed = false;
        }
        int nparts = 0;
        e = qmm::launch_gemv_argmax(t.type, mat_args(t, 1, K, seed ? nullptr : scan), xk, x0, round16, ids, id_limit,
                                    mine, &nparts, ctx->stream, pre, true, pend->x32, pend->gamma);
        if (e == hipSuccess) {
            pend->on = true;
            pend->part = mine;
            pend->nparts = nparts;
            pend->row_base = row_base;
            pend->thresh = step->thresh;
            pend->checkpoint = step->checkpoint;
            pend->c = step->c;
            return QMM_OK;
        }
        if (e != hipErrorNotSupported || seed || pend->x32) return hip_fail(ctx, e, "GEMV + argmax launch");
        int rc = launch_pending(ctx, *pend, best_val, best_id, *step, scan);
        if (rc) return rc;
    } else if (M == 1) {  // the GEMV's persistent grid reduces to one partial per workgroup
        int nparts = 0;
        e = qmm::launch_gemv_argmax(t.type, mat_args(t, 1, K, scan), xk, x0, round16, ids, id_limit, part, &nparts,
                                    ctx->stream);
        if (e == hipSuccess) {
            e = step ? qmm::launch_scan_final(part, nparts, row_base, best_val, best_id, step->cand, step->draft,
                                              step->margin, step->thresh, step->checkpoint, step->c, scan, ctx->stream)
                     : qmm::launch_argmax_final(part, nparts, ids, row_base, best_val, best_id, scan, ctx->stream);
            return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "argmax launch");
        }
        if (e != hipErrorNotSupported) return hip_fail(ctx, e, "GEMV + argmax launch");
    }
    int rc = run_tasks(ctx, nullptr, q8k, q80, M, K, &t, 1, scan);
    if (rc) return rc;
    if (step) {
        e = qmm::launch_argmax_partials(logits, M, rows, size_t(rows), part, scan, ctx->stream);
        if (e == hipSuccess)
            e = qmm::launch_scan_final(part, qmm::argmax_slices(rows), row_base, best_val, best_id, step->cand,
                                       step->draft, step->margin, step->thresh, step->checkpoint, step->c, scan,
                                       ctx->stream);
    } else {
        e = qmm::launch_argmax(logits, M, rows, size_t(rows), round16, ids, id_limit, row_base, best_val, best_id, part,
                               scan, ctx->stream);
    }
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "argmax launch");
}

int lm_argmax(qmm_context *ctx, const void *q8k, const void *q80, int M, int K, const void *w, uint32_t type,
              int rows, uint32_t row_base, const uint32_t *ids, uint32_t id_limit, float *logits_out, float *best_val,
              uint32_t *best_id) {
    if (!ctx) return QMM_EINVAL;
    if (!best_val || !best_id) return fail(ctx, QMM_EINVAL, "bad LM-head arguments");
    if (!aligned(best_val, 4) || !aligned(best_id, 4) || (logits_out && !aligned(logits_out, 4)))
        return fail(ctx, QMM_EALIGN, "best_val/best_id/logits must be 4-B aligned");
    qmm_matrix_task t;
    int rc = lm_task(ctx, q8k, q80, M, K, w, type, rows, logits_out, t);
    if (rc) return rc;
    if ((rc = use_device(ctx))) return rc;
    const LmScratch L = lm_scratch(M, rows, t.row_bytes, logits_out != nullptr, ids != nullptr);
    if ((rc = ensure_lm(ctx, L.total()))) return rc;
    return lm_argmax_run(ctx, q8k, q80, M, K, t, row_base, ids, id_limit, logits_out, best_val, best_id,
                         static_cast<uint8_t *>(ctx->lm), nullptr, nullptr);
}

}  // namespace

extern "C" {

const char *qmm_status_string(int status) {
    switch (status) {
        case QMM_OK: return "ok";
        case QMM_EINVAL: return "invalid argument";
        case QMM_ETYPE: return "unsupported ggml type";
        case QMM_ESHAPE: return "shape mismatch";
        case QMM_EHIP: return "HIP runtime error";
        case QMM_ENOMEM: return "device allocation failed";
        case QMM_EALIGN: return "misaligned device pointer";
        case QMM_ENOTFOUND: return "tensor not found";
        default: return "unknown status";
    }
}

const char *qmm_last_error(const qmm_context *ctx) { return ctx ? ctx->err.c_str() : ""; }

size_t qmm_row_bytes(uint32_t type, int64_t cols) {
    if (!supported(type) || cols <= 0 || cols % block_values(type)) return 0;
    switch (type) {
        case qmm::kF32: return size_t(cols) * 4;
        case qmm::kF16: return size_t(cols) * 2;
        case qmm::kQ8_0: return size_t(cols / 32) * 34;
        case qmm::kQ4_K: return size_t(cols / 256) * 144;
        case qmm::kQ5_K: return size_t(cols / 256) * 176;
        case qmm::kQ6_K: return size_t(cols / 256) * 210;
    }
    return 0;
}

size_t qmm_q8k_bytes(int M, int K) { return (M > 0 && K > 0) ? qmm::Q8KLayout(M, K).total : 0; }
size_t qmm_q8k_d_offset(int M, int K) { return (M > 0 && K > 0) ? qmm::Q8KLayout(M, K).d_off : 0; }
size_t qmm_q8k_bsum_offset(int M, int K) { return (M > 0 && K > 0) ? qmm::Q8KLayout(M, K).bs_off : 0; }
size_t qmm_q8k_tile_offset(int M, int K) { return (M > 0 && K > 0) ? qmm::Q8KLayout(M, K).tile_off : 0; }
size_t qmm_q8k_h_offset(int M, int K) { return (M > 0 && K > 0) ? qmm::Q8KLayout(M, K).h_off : 0; }
size_t qmm_q8k_bh_offset(int M, int K) { return (M > 0 && K > 0) ? qmm::Q8KLayout(M, K).bh_off : 0; }
size_t qmm_q8_0_bytes(int M, int K) { return (M > 0 && K > 0) ? qmm::Q80Layout(M, K).total : 0; }
size_t qmm_q8_0_d_offset(int M, int K) { return (M > 0 && K > 0) ? qmm::Q80Layout(M, K).d_off : 0; }

int qmm_init(int device, qmm_context **out_ctx) {
    if (!out_ctx) return QMM_EINVAL;
    *out_ctx = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return QMM_EHIP;
    }
    if (device < 0 || device >= n) return QMM_EINVAL;
    qmm_context *ctx = new qmm_context();
    ctx->device = device;
    if ((e = hipSetDevice(device)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreate(&ctx->ev0)) != hipSuccess ||
        (e = hipEventCreate(&ctx->ev1)) != hipSuccess) {
        delete ctx;
        return QMM_EHIP;
    }
    // the device address of `scratch`, looked up once per device with that
    // device current; a failed lookup disables only the no-allocation entry
    if (device < kMaxDevices) {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (!g_scratch_on[device]) {
            void *ptr = nullptr;
            e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
            if (e == hipSuccess && ptr) g_scratch_on[device] = ptr;
            else {
                (void)hipGetLastError();
                ctx->scratch_err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
            }
        }
        ctx->scratch = g_scratch_on[device];
    } else {
        ctx->scratch_err = "device index beyond the scratch table";
    }
    ctx->stream = ctx->own_stream;
    *out_ctx = ctx;
    return QMM_OK;
}

int qmm_destroy(qmm_context *ctx) {
    if (!ctx) return QMM_EINVAL;
    (void)use_device(ctx);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->act) (void)hipFree(ctx->act);
    if (ctx->lm) (void)hipFree(ctx->lm);
    if (ctx->fold) (void)hipFree(ctx->fold);
    for (void *p : ctx->retired) (void)hipFree(p);
    if (ctx->ev0) (void)hipEventDestroy(ctx->ev0);
    if (ctx->ev1) (void)hipEventDestroy(ctx->ev1);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return QMM_OK;
}

int qmm_set_stream(qmm_context *ctx, void *hip_stream) {
    if (!ctx) return QMM_EINVAL;
    ctx->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own_stream;
    return QMM_OK;
}

void *qmm_get_stream(qmm_context *ctx) { return ctx ? static_cast<void *>(ctx->stream) : nullptr; }

int qmm_synchronize(qmm_context *ctx) {
    if (!ctx) return QMM_EINVAL;
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "hipStreamSynchronize");
}

int qmm_reserve(qmm_context *ctx, int max_M, int max_K) {
    if (!ctx || max_M <= 0 || max_K <= 0) return fail(ctx, QMM_EINVAL, "bad reserve size");
    int rc = use_device(ctx);
    if (rc) return rc;
    (void)ensure_fold(ctx);  // (small; a later scan retries where this fails)
    return ensure_act(ctx, std::max(qmm::Q8KLayout(max_M, max_K).total + qmm::Q80Layout(max_M, max_K).total,
                                    ffn_scratch_bytes(max_K)));
}

int qmm_device_info(qmm_context *ctx, int *cu_count, size_t *hbm_bytes, char *arch, size_t arch_len) {
    if (!ctx) return QMM_EINVAL;
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, ctx->device);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGetDeviceProperties");
    if (cu_count) *cu_count = p.multiProcessorCount;
    if (hbm_bytes) *hbm_bytes = p.totalGlobalMem;
    if (arch && arch_len) {
        std::snprintf(arch, arch_len, "%s", p.gcnArchName);
    }
    return QMM_OK;
}

int qmm_malloc(qmm_context *ctx, size_t bytes, void **dev_ptr) {
    if (!ctx || !dev_ptr || bytes == 0) return fail(ctx, QMM_EINVAL, "bad malloc arguments");
    *dev_ptr = nullptr;
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = hipMalloc(dev_ptr, bytes);
    if (e != hipSuccess) {
        *dev_ptr = nullptr;
        (void)hipGetLastError();
        return fail(ctx, QMM_ENOMEM, "hipMalloc failed");
    }
    return QMM_OK;
}

int qmm_free(qmm_context *ctx, void *dev_ptr) {
    if (!ctx) return QMM_EINVAL;
    if (!dev_ptr) return QMM_OK;
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = hipFree(dev_ptr);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "hipFree");
}

int qmm_memcpy_h2d(qmm_context *ctx, void *dst_dev, const void *src_host, size_t bytes) {
    if (!ctx || (bytes && (!dst_dev || !src_host))) return fail(ctx, QMM_EINVAL, "bad memcpy arguments");
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "hipMemcpy H2D");
}

int qmm_memcpy_d2h(qmm_context *ctx, void *dst_host, const void *src_dev, size_t bytes) {
    if (!ctx || (bytes && (!dst_host || !src_dev))) return fail(ctx, QMM_EINVAL, "bad memcpy arguments");
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "hipMemcpy D2H");
}

int qmm_memcpy_d2d(qmm_context *ctx, void *dst_dev, const void *src_dev, size_t bytes) {
    if (!ctx || (bytes && (!dst_dev || !src_dev))) return fail(ctx, QMM_EINVAL, "bad memcpy arguments");
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(dst_dev, src_dev, bytes, hipMemcpyDeviceToDevice, ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "hipMemcpy D2D");
}

int qmm_weight_upload(qmm_context *ctx, const void *host_blocks, uint32_t type, int64_t rows,
                      int64_t cols, void **dev_blocks) {
    if (!ctx || !host_blocks || !dev_blocks || rows <= 0) return fail(ctx, QMM_EINVAL, "bad upload arguments");
    *dev_blocks = nullptr;
    if (!supported(type)) return fail(ctx, QMM_ETYPE, "unsupported ggml type");
    const size_t rb = qmm_row_bytes(type, cols);
    if (!rb) return fail(ctx, QMM_ESHAPE, "cols not a multiple of the block size");
    const size_t bytes = rb * size_t(rows);
    void *p = nullptr;
    int rc = qmm_malloc(ctx, qmm::align256(bytes) + 256, &p);
    if (rc) return rc;
    rc = qmm_memcpy_h2d(ctx, p, host_blocks, bytes);
    if (rc) {
        (void)hipFree(p);
        return rc;
    }
    *dev_blocks = p;
    return QMM_OK;
}

int qmm_quantize_q8k(qmm_context *ctx, const float *x, int M, int K, void *q8k_out) {
    if (!ctx) return QMM_EINVAL;
    if (!x || !q8k_out || M <= 0 || K <= 0) return fail(ctx, QMM_EINVAL, "bad quantize arguments");
    if (K % 256) return fail(ctx, QMM_ESHAPE, "K must be a multiple of 256 for Q8_K");
    if (!aligned(x, 16) || !aligned(q8k_out, 16)) return fail(ctx, QMM_EALIGN, "x and the Q8_K buffer must be 16-B aligned");
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = qmm::launch_quantize_q8k(x, M, K, q8k_out, ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "quantize_q8k launch");
}

int qmm_quantize_q8_0(qmm_context *ctx, const float *x, int M, int K, void *q80_out) {
    if (!ctx) return QMM_EINVAL;
    if (!x || !q80_out || M <= 0 || K <= 0) return fail(ctx, QMM_EINVAL, "bad quantize arguments");
    if (K % 32) return fail(ctx, QMM_ESHAPE, "K must be a multiple of 32 for Q8_0");
    if (!aligned(x, 16) || !aligned(q80_out, 16)) return fail(ctx, QMM_EALIGN, "x and the Q8_0 buffer must be 16-B aligned");
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = qmm::launch_quantize_q8_0(x, M, K, q80_out, ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "quantize_q8_0 launch");
}

int qmm_swiglu_q8k(qmm_context *ctx, const float *gate, const float *up, int M, int N, float *h_out,
                   void *q8k_out) {
    if (!ctx) return QMM_EINVAL;
    if (!gate || !up || !q8k_out || M <= 0 || N <= 0) return fail(ctx, QMM_EINVAL, "bad swiglu arguments");
    if (N % 256) return fail(ctx, QMM_ESHAPE, "N must be a multiple of 256");
    if (!aligned(gate, 16) || !aligned(up, 16) || !aligned(q8k_out, 16) || (h_out && !aligned(h_out, 16)))
        return fail(ctx, QMM_EALIGN, "swiglu buffers must be 16-B aligned");
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = qmm::launch_swiglu_q8k(gate, up, M, N, h_out, q8k_out, ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "swiglu launch");
}

int qmm_rmsnorm_q8k(qmm_context *ctx, const float *x, const float *gamma, int M, int K, float *y_out,
                    void *q8k_out) {
    if (!ctx) return QMM_EINVAL;
    if (!x || !gamma || !q8k_out || M <= 0 || K <= 0) return fail(ctx, QMM_EINVAL, "bad rmsnorm arguments");
    if (K % 256) return fail(ctx, QMM_ESHAPE, "K must be a multiple of 256");
    if (K > 16384) return fail(ctx, QMM_ESHAPE, "K above 16384");
    if (!aligned(x, 16) || !aligned(gamma, 16) || !aligned(q8k_out, 16) || (y_out && !aligned(y_out, 16)))
        return fail(ctx, QMM_EALIGN, "rmsnorm buffers must be 16-B aligned");
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = qmm::launch_rmsnorm_q8k(x, gamma, M, K, y_out, q8k_out, ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "rmsnorm launch");
}

namespace {

// qmm_ffn_block, and with gamma (x then the row before its RMSNorm) the
// block behind its input norm
int ffn_block(qmm_context *ctx, const float *x, const float *gamma, const void *q8k, int K, qmm_matrix_task *gate,
              qmm_matrix_task *up, qmm_matrix_task *down, float *h_out) {
    if (!gate || !up || !down) return fail(ctx, QMM_EINVAL, "null task");
    if ((x == nullptr) == (q8k == nullptr)) return fail(ctx, QMM_EINVAL, "give exactly one of x and q8k");
    qmm_matrix_task gu[2] = {*gate, *up};
    bool need_q8k, need_q80;
    int rc = check_tasks(ctx, 1, K, gu, 2, &need_q8k, &need_q80);
    if (rc) return rc;
    const int N = gate->rows;
    if (N <= 0 || up->rows != N || up->type != gate->type)
        return fail(ctx, QMM_ESHAPE, "gate and up must have the same positive rows and type");
    if (N % 256) return fail(ctx, QMM_ESHAPE, "gate/up rows must be a multiple of 256 (h is quantized to Q8_K)");
    if (x && !aligned(x, 16)) return fail(ctx, QMM_EALIGN, "x must be 16-B aligned");
    if (q8k && (rc = check_pre(ctx, q8k, nullptr, need_q8k, need_q80))) return rc;
    if (!aligned(gate->dst, 16) || !aligned(up->dst, 16) || (h_out && !aligned(h_out, 16)))
        return fail(ctx, QMM_EALIGN, "gate/up outputs and h_out must be 16-B aligned");
    qmm_matrix_task dn = *down;
    bool dn_q8k, dn_q80;
    if ((rc = check_tasks(ctx, 1, N, &dn, 1, &dn_q8k, &dn_q80))) return rc;
    if (dn_q80) return fail(ctx, QMM_ETYPE, "a Q8_0 down task needs Q8_0 activations; h is quantized to Q8_K");
    if ((rc = use_device(ctx))) return rc;
    // (with the norm, the normed row's Q8_K behind the block's scratch, for the three-step form)
    const size_t norm_b = gamma ? align256(qmm::Q8KLayout(1, K).total) : 0;
    if ((rc = ensure_act(ctx, ffn_scratch_bytes(N) + norm_b))) return rc;
    uint8_t *scr = static_cast<uint8_t *>(ctx->act);
    void *hq = scr;  // h's Q8_K (separate launches) or h in fp16 (one launch)
    float *h = h_out ? h_out : reinterpret_cast<float *>(scr + align256(qmm::Q8KLayout(1, N).total));
    qmm::Q8KView xk;
    qmm::Q80View x0;
    act_views(q8k, nullptr, 1, K, xk, x0);
    // two launches where they apply: gate/up with SwiGLU in its epilogue,
    // then the down GEMV on h in fp16
    const qmm::MatArgs da = mat_args(dn, 1, N);
    uint32_t *hx = static_cast<uint32_t *>(hq);
    if ((gate->type == qmm::kQ4_K || gate->type == qmm::kQ5_K) && dn.rows > 0 && K % 256 == 0 && K <= 3072 &&
        N <= 12288 &&
        qmm::launch_gemv_x16(dn.type, da, reinterpret_cast<const uint16_t *>(hx), ctx->stream, false) == hipSuccess) {
        qmm::FfnArgs a{};
        a.wg = static_cast<const uint8_t *>(gate->w_base);
        a.wu = static_cast<const uint8_t *>(up->w_base);
        a.g = gate->dst;
        a.u = up->dst;
        a.h_out = h_out;
        a.hx = hx;
        a.K = K;
        a.F = N;
        a.rb1 = int(gate->row_bytes);
        a.type = gate->type;
        a.gamma = gamma;
        hipError_t e = qmm::launch_ffn_gate_up(a, x, xk, ctx->stream);
        if (e == hipSuccess) e = qmm::launch_gemv_x16(dn.type, da, reinterpret_cast<const uint16_t *>(hx), ctx->stream);
        return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "FFN block launch");
    }
    // the reference's three steps as separate launches (after the norm's own)
    if (gamma) {
        void *nq = scr + ffn_scratch_bytes(N);
        const hipError_t e = qmm::launch_rmsnorm_q8k(x, gamma, 1, K, nullptr, nq, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "rmsnorm launch");
        x = nullptr;
        q8k = nq;
    }
    if ((rc = run_tasks(ctx, x, q8k, nullptr, 1, K, gu, 2))) return rc;
    const hipError_t e = qmm::launch_swiglu_q8k(gate->dst, up->dst, 1, N, h, hq, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "swiglu launch");
    return run_tasks(ctx, nullptr, hq, nullptr, 1, N, &dn, 1);
}

}  // namespace

int qmm_ffn_block(qmm_context *ctx, const float *x, const void *q8k, int K, qmm_matrix_task *gate,
                  qmm_matrix_task *up, qmm_matrix_task *down, float *h_out) {
    if (!ctx) return QMM_EINVAL;
    return ffn_block(ctx, x, nullptr, q8k, K, gate, up, down, h_out);
}

int qmm_ffn_block_rmsnorm(qmm_context *ctx, const float *x, const float *gamma, int K, qmm_matrix_task *gate,
                          qmm_matrix_task *up, qmm_matrix_task *down, float *h_out) {
    if (!ctx) return QMM_EINVAL;
    if (!x || !gamma) return fail(ctx, QMM_EINVAL, "null x or gamma");
    if (K % 256) return fail(ctx, QMM_ESHAPE, "K must be a multiple of 256");
    if (K > 16384) return fail(ctx, QMM_ESHAPE, "K above 16384");
    if (!aligned(gamma, 16)) return fail(ctx, QMM_EALIGN, "gamma must be 16-B aligned");
    return ffn_block(ctx, x, gamma, nullptr, K, gate, up, down, h_out);
}

int qmm_dequantize_f16(qmm_context *ctx, const void *w_blocks, uint32_t type, int64_t rows,
                       int64_t cols, uint16_t *dst) {
    if (!ctx) return QMM_EINVAL;
    if (!w_blocks || !dst || rows <= 0 || cols <= 0) return fail(ctx, QMM_EINVAL, "bad dequantize arguments");
    if (!supported(type)) return fail(ctx, QMM_ETYPE, "unsupported ggml type");
    if (cols % block_values(type)) return fail(ctx, QMM_ESHAPE, "cols not a multiple of the block size");
    if (!aligned(dst, 2)) return fail(ctx, QMM_EALIGN, "dst must be 2-B aligned");
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = qmm::launch_dequant_f16(static_cast<const uint8_t *>(w_blocks), type, rows, cols,
                                           dst, ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "dequantize launch");
}

int qmm_gemm_multi_dispatch(qmm_context *ctx, const float *x, int M, int K, qmm_matrix_task *tasks,
                            int n_tasks) {
    if (!ctx) return QMM_EINVAL;
    if (!x) return fail(ctx, QMM_EINVAL, "null x");
    bool need_q8k, need_q80;
    int rc = check_tasks(ctx, M, K, tasks, n_tasks, &need_q8k, &need_q80);
    if (rc) return rc;
    if (!aligned(x, 16)) return fail(ctx, QMM_EALIGN, "x must be 16-B aligned");
    if ((rc = use_device(ctx))) return rc;
    if (M == 1) return run_tasks(ctx, x, nullptr, nullptr, M, K, tasks, n_tasks);
    hipError_t e;
    // 2..4 tokens, one k-quant task in the batch-1 GEMV's shape: the kernel
    // quantizes the rows in its fill (no quantizer launch), as at batch 1
    if (M <= 4) {
        int live = -1, nlive = 0;
        for (int t = 0; t < n_tasks; ++t)
            if (tasks[t].rows > 0) {
                live = t;
                ++nlive;
            }
        if (nlive == 1 && !need_q80 && !is_float(tasks[live].type)) {
            const qmm::MatArgs a = mat_args(tasks[live], M, K);
            if (qmm::gemv_mt_shape(a)) {
                e = qmm::launch_gemv_mt(tasks[live].type, &a, 1, qmm::Q8KView{}, ctx->stream, x);
                if (e == hipSuccess) return QMM_OK;
                if (e != hipErrorNotSupported) return hip_fail(ctx, e, "matmul launch");
            }
        }
    }
    const size_t k_bytes = need_q8k ? qmm::Q8KLayout(M, K).total : 0;
    const size_t z_bytes = need_q80 ? qmm::Q80Layout(M, K).total : 0;
    if ((rc = ensure_act(ctx, k_bytes + z_bytes))) return rc;
    void *q8k = need_q8k ? ctx->act : nullptr;
    void *q80 = need_q80 ? static_cast<uint8_t *>(ctx->act) + k_bytes : nullptr;
    if (need_q8k && (e = qmm::launch_quantize_q8k(x, M, K, q8k, ctx->stream, q8k_skip(M, tasks, n_tasks))) !=
                        hipSuccess)
        return hip_fail(ctx, e, "quantize_q8k launch");
    if (need_q80 && (e = qmm::launch_quantize_q8_0(x, M, K, q80, ctx->stream)) != hipSuccess)
        return hip_fail(ctx, e, "quantize_q8_0 launch");
    return run_tasks(ctx, nullptr, q8k, q80, M, K, tasks, n_tasks);
}

int qmm_gemm_multi_dispatch_rmsnorm(qmm_context *ctx, const float *x, const float *gamma, int M, int K,
                                    qmm_matrix_task *tasks, int n_tasks) {
    if (!ctx) return QMM_EINVAL;
    if (!x || !gamma) return fail(ctx, QMM_EINVAL, "null x or gamma");
    bool need_q8k, need_q80;
    int rc = check_tasks(ctx, M, K, tasks, n_tasks, &need_q8k, &need_q80);
    if (rc) return rc;
    if (K % 256) return fail(ctx, QMM_ESHAPE, "K must be a multiple of 256");
    if (K > 16384) return fail(ctx, QMM_ESHAPE, "K above 16384");
    if (!aligned(x, 16) || !aligned(gamma, 16)) return fail(ctx, QMM_EALIGN, "x and gamma must be 16-B aligned");
    if ((rc = use_device(ctx))) return rc;
    // batch 1, k-quant tasks: the norm inside every workgroup's activation fill
    if (M == 1 && !need_q80) {
        qmm::MatArgs group[qmm::kMaxGroup];
        int n = 0;
        bool fits = true;
        for (int t = 0; t < n_tasks && fits; ++t) {
            if (tasks[t].rows == 0) continue;
            if (n == qmm::kMaxGroup || is_float(tasks[t].type)) fits = false;
            else group[n++] = mat_args(tasks[t], 1, K);
        }
        if (fits && n > 0) {
            const hipError_t e = qmm::launch_gemv_rms(group, n, x, gamma, ctx->stream);
            if (e == hipSuccess) return QMM_OK;
            if (e != hipErrorNotSupported) return hip_fail(ctx, e, "matmul launch");
        }
    }
    // else the norm's own kernel into the context's buffers, then the tasks
    const size_t k_bytes = qmm::Q8KLayout(M, K).total;
    const size_t y_bytes = need_q80 ? align256(size_t(M) * size_t(K) * 4) : 0;
    const size_t z_bytes = need_q80 ? qmm::Q80Layout(M, K).total : 0;
    if ((rc = ensure_act(ctx, k_bytes + y_bytes + z_bytes))) return rc;
    uint8_t *base = static_cast<uint8_t *>(ctx->act);
    float *y = need_q80 ? reinterpret_cast<float *>(base + k_bytes) : nullptr;
    void *q80 = need_q80 ? base + k_bytes + y_bytes : nullptr;
    hipError_t e = qmm::launch_rmsnorm_q8k(x, gamma, M, K, y, base, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "rmsnorm launch");
    if (need_q80 && (e = qmm::launch_quantize_q8_0(y, M, K, q80, ctx->stream)) != hipSuccess)
        return hip_fail(ctx, e, "quantize_q8_0 launch");
    return run_tasks(ctx, nullptr, base, q80, M, K, tasks, n_tasks);
}

int qmm_gemm_multi_dispatch_noalloc(qmm_context *ctx, const float *x, int M, int K, qmm_matrix_task *tasks,
                                    int n_tasks) {
    if (!ctx) return QMM_EINVAL;
    if (!x) return fail(ctx, QMM_EINVAL, "null x");
    bool need_q8k, need_q80;
    int rc = check_tasks(ctx, M, K, tasks, n_tasks, &need_q8k, &need_q80);
    if (rc) return rc;
    if (!aligned(x, 16)) return fail(ctx, QMM_EALIGN, "x must be 16-B aligned");
    if (M == 1) {  // the batch-1 kernels quantize x themselves: no scratch
        if ((rc = use_device(ctx))) return rc;
        return run_tasks(ctx, x, nullptr, nullptr, M, K, tasks, n_tasks);
    }
    const size_t k_bytes = need_q8k ? qmm::Q8KLayout(M, K).total : 0;
    const size_t z_bytes = need_q80 ? qmm::Q80Layout(M, K).total : 0;
    if (k_bytes + z_bytes > kScratchBytes)
        return fail(ctx, QMM_ESHAPE,
                    "the quantized input of M x K = " + std::to_string(M) + " x " + std::to_string(K) + " needs " +
                        std::to_string(k_bytes + z_bytes) + " bytes, more than the " + std::to_string(kScratchBytes) +
                        "-byte device scratch of the no-allocation dispatch");
    if (!ctx->scratch) return fail(ctx, QMM_EHIP, "no device scratch: " + ctx->scratch_err);
    if ((rc = use_device(ctx))) return rc;
    uint8_t *base = static_cast<uint8_t *>(ctx->scratch);
    void *q8k = need_q8k ? base : nullptr;
    void *q80 = need_q80 ? base + k_bytes : nullptr;  // (k_bytes is a multiple of 256)
    hipError_t e;
    if (need_q8k && (e = qmm::launch_quantize_q8k(x, M, K, q8k, ctx->stream, q8k_skip(M, tasks, n_tasks))) !=
                        hipSuccess)
        return hip_fail(ctx, e, "quantize_q8k launch");
    if (need_q80 && (e = qmm::launch_quantize_q8_0(x, M, K, q80, ctx->stream)) != hipSuccess)
        return hip_fail(ctx, e, "quantize_q8_0 launch");
    return run_tasks(ctx, nullptr, q8k, q80, M, K, tasks, n_tasks);
}

size_t qmm_noalloc_scratch_bytes(void) { return kScratchBytes; }

int qmm_gemm_multi_dispatch_prequantized(qmm_context *ctx, const void *q8k, const void *q80, int M,
                                         int K, qmm_matrix_task *tasks, int n_tasks) {
    if (!ctx) return QMM_EINVAL;
    bool need_q8k, need_q80;
    int rc = check_tasks(ctx, M, K, tasks, n_tasks, &need_q8k, &need_q80);
    if (rc) return rc;
    if ((rc = check_pre(ctx, q8k, q80, need_q8k, need_q80))) return rc;
    if ((rc = use_device(ctx))) return rc;
    return run_tasks(ctx, nullptr, need_q8k ? q8k : nullptr, need_q80 ? q80 : nullptr, M, K, tasks,
                     n_tasks);
}

int qmm_lm_head_argmax(qmm_context *ctx, const void *q8k, const void *q80, int M, int K, const void *w_rows,
                       uint32_t type, int rows, uint32_t row_base, float *logits_out, float *best_val,
                       uint32_t *best_id) {
    return lm_argmax(ctx, q8k, q80, M, K, w_rows, type, rows, row_base, nullptr, 0u, logits_out, best_val, best_id);
}

int qmm_eval_rows_argmax(qmm_context *ctx, const void *q8k, const void *q80, int M, int K, const void *w_tensor,
                         int64_t tensor_rows, uint32_t type, const uint32_t *row_ids, int n_ids, float *vals_out,
                         float *best_val, uint32_t *best_id) {
    if (!ctx) return QMM_EINVAL;
    if (!row_ids) return fail(ctx, QMM_EINVAL, "row_ids is NULL");
    if (tensor_rows <= 0 || tensor_rows > int64_t(UINT32_MAX)) return fail(ctx, QMM_EINVAL, "bad tensor_rows");
    return lm_argmax(ctx, q8k, q80, M, K, w_tensor, type, n_ids, 0, row_ids, uint32_t(tensor_rows), vals_out, best_val,
                     best_id);
}

// The scan over quantized activations (q8k / q80), or, with x32, over the
// row before its RMSNorm (gamma): at batch 1 with nothing evaluated ahead of
// the chunks and every chunk launch on the fused argmax grid, each launch
// normalizes the row in its fill; otherwise the norm's own kernel first
// writes q8k (and, for a Q8_0 tensor, y and q80).
static int lm_scan(qmm_context *ctx, const void *q8k, const void *q80, const float *x32, const float *gamma, float *y,
                   int M, int K, const void *w_lm, uint32_t type, int vocab_rows, const qmm_lm_scan_params *params,
                   const uint32_t *pre_ids, int n_pre, const uint32_t *draft_ids, float *best_val, uint32_t *best_id,
                   int32_t *scan_state) {
    if (!params || !best_val || !best_id || !scan_state || vocab_rows <= 0 || M <= 0 || n_pre < 0 ||
        (n_pre > 0 && !pre_ids))
        return fail(ctx, QMM_EINVAL, "bad LM-head scan arguments");
    if (params->chunk_rows <= 0 || params->n_thresholds < 0 || (params->n_thresholds > 0 && !params->thresholds) ||
        params->first_checkpoint < 0)
        return fail(ctx, QMM_EINVAL, "bad LM-head scan parameters");
    if (!aligned(best_val, 4) || !aligned(best_id, 4) || !aligned(scan_state, 4))
        return fail(ctx, QMM_EALIGN, "best_val/best_id/scan_state must be 4-B aligned");
    const int nchunks = (vocab_rows + params->chunk_rows - 1) / params->chunk_rows;
    // this call's chunks [cb, ce); a resumed scan seeds nothing
    const int cb = params->chunk_begin, ce = params->chunk_end ? params->chunk_end : nchunks;
    const bool resume = params->resume != 0;
    if (cb < 0 || ce < cb || ce > nchunks) return fail(ctx, QMM_EINVAL, "bad LM-head scan chunk range");
    // Chunks share a launch up to the next chunk after which something is
    // decided: a checkpoint (E:11248-11256), with drafts the pruning
    // (E:11203-11209, after every chunk), or the call's last chunk. In
    // between nothing changes the scan's course, and the strict running
    // update over the merged rows (the first row holding the largest value,
    // if it beats the best) is the chunk-by-chunk updates' result.
    const bool prunes = draft_ids && M >= 2;
    auto decides = [&](int c) {
        return prunes || c == ce - 1 || (params->n_thresholds > 0 && c >= params->first_checkpoint);
    };
    std::vector<std::pair<int, int>> groups;  // [first chunk, last chunk] of each launch
    int chunk = std::min(params->chunk_rows, vocab_rows);  // rows of the largest launch
    for (int c0 = cb; c0 < ce;) {
        int c1 = c0;
        while (!decides(c1)) ++c1;
        groups.emplace_back(c0, c1);
        const int64_t end = std::min<int64_t>(int64_t(c1 + 1) * params->chunk_rows, vocab_rows);
        chunk = std::max(chunk, int(end - int64_t(c0) * params->chunk_rows));
        c0 = c1 + 1;
    }
    // validate every launch's task before the first launch
    qmm_matrix_task tc, tp, td;
    int rc = lm_task(ctx, q8k, q80, M, K, w_lm, type, chunk, nullptr, tc);
    if (!rc && n_pre > 0) rc = lm_task(ctx, q8k, q80, M, K, w_lm, type, n_pre, nullptr, tp);
    if (!rc && draft_ids && M >= 2) rc = lm_task(ctx, q8k, q80, M, K, w_lm, type, M - 1, nullptr, td);
    if (rc) return rc;
    if ((rc = use_device(ctx))) return rc;
    // scratch: candidate logits [M] | candidate dots [M][M - 1] | the largest call's area
    const size_t rb = tc.row_bytes;
    const size_t cand_b = align256(size_t(M) * 4), cdot_b = align256(size_t(M) * size_t(std::max(M - 1, 1)) * 4);
    const size_t part_b = lm_scratch(M, chunk, rb, false, false).part_b;
    size_t area = lm_scratch(M, chunk, rb, false, false).total() + (M == 1 ? 2 * part_b : 0);
    if (n_pre > 0) area = std::max(area, lm_scratch(M, n_pre, rb, false, true).total());
    if (draft_ids && M >= 2) area = std::max(area, align256(size_t(M - 1) * rb));
    if ((rc = ensure_lm(ctx, cand_b + cdot_b + area))) return rc;
    uint8_t *scr = static_cast<uint8_t *>(ctx->lm);
    float *cand = reinterpret_cast<float *>(scr);
    float *cdot = reinterpret_cast<float *>(scr + cand_b);
    uint8_t *work = scr + cand_b + cdot_b;
    const uint8_t *wb = static_cast<const uint8_t *>(w_lm);
    PendingStep pend;
    hipError_t e;
    // At batch 1 with nothing evaluated ahead of the chunks, the first chunk's
    // launch seeds the scan's state (where it takes the fused argmax grid)
    // instead of a launch of its own.
    {
        qmm::Q8KView xk;
        qmm::Q80View x0;
        act_views(q8k, q80, 1, K, xk, x0);
        auto fused = [&](const std::pair<int, int> &gr, const float *g, int &np) {
            qmm_matrix_task t = tc;
            const int r0 = gr.first * params->chunk_rows;
            t.rows = int(std::min<int64_t>(int64_t(gr.second + 1) * params->chunk_rows, vocab_rows) - r0);
            np = 0;
            return qmm::launch_gemv_argmax(t.type, mat_args(t, 1, K), xk, x0, true, nullptr, 0u, nullptr, &np,
                                           ctx->stream, qmm::PrevStep{}, false, x32, g) == hipSuccess;
        };
        int np = 0;
        const bool first_fused = M == 1 && n_pre == 0 && !groups.empty() && fused(groups[0], nullptr, np);
        pend.seed = first_fused && !resume;
        bool normed = x32 && first_fused;
        // every launch after the first reads its predecessor's per-workgroup
        // partials, at most 1024 of them (the bound each launch applies to
        // its PrevStep): where a launch's grid has more, the scan takes the
        // norm's own launch, before anything is enqueued
        for (size_t i = 0; i < groups.size() && normed; ++i) {
            const int prev = np;
            normed = (i == 0 || prev <= 1024) && fused(groups[i], gamma, np);
        }
        if (normed) {
            pend.x32 = x32;
            pend.gamma = gamma;
        } else if (x32) {  // the norm's own launch, into q8k (and y, q80 for a Q8_0 tensor)
            e = qmm::launch_rmsnorm_q8k(x32, gamma, M, K, q80 ? y : nullptr, const_cast<void *>(q8k), ctx->stream);
            if (e != hipSuccess) return hip_fail(ctx, e, "rmsnorm launch");
            if (q80 && (e = qmm::launch_quantize_q8_0(y, M, K, const_cast<void *>(q80), ctx->stream)) != hipSuccess)
                return hip_fail(ctx, e, "quantize_q8_0 launch");
        }
    }
    if (!pend.seed && !resume) {
        e = qmm::launch_scan_init(M, best_val, best_id, cand, scan_state, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "scan init launch");
    }
    // the rows every active position evaluates first, fp32, in list order:
    // the end-of-text rows of a new scan (E:11143-11146, every position
    // active), the extended-script rows of a resumed one (E:11216-11225)
    if (n_pre > 0 && (rc = lm_argmax_run(ctx, q8k, q80, M, K, tp, 0, pre_ids, uint32_t(vocab_rows), nullptr, best_val,
                                         best_id, work, scan_state, nullptr)))
        return rc;
    // each position's draft candidate (E:11147-11153). A resumed scan
    // derives the candidates' logits again (the pruning needs them); their
    // strict update changes nothing, as every position's best already
    // includes its candidate. Then, after the extended rows, the pruning
    // rule once (E:11226-11231).
    if (draft_ids && M >= 2) {
        e = qmm::launch_gather_rows(wb, rb, draft_ids + 1, uint32_t(vocab_rows), M - 1, work, nullptr, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "row gather launch");
        td.w_base = work;
        td.dst = cdot;
        if ((rc = run_tasks(ctx, nullptr, q8k, q80, M, K, &td, 1))) return rc;
        e = qmm::launch_scan_cand(M, cdot, draft_ids, uint32_t(vocab_rows), best_val, best_id, cand, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "candidate launch");
        if (resume) {
            e = qmm::launch_scan_final(nullptr, 0, 0u, best_val, best_id, cand, draft_ids, params->prune_margin, -1e30f,
                                       false, cb - 1, scan_state, ctx->stream);
            if (e != hipSuccess) return hip_fail(ctx, e, "pruning launch");
        }
    }
    // the chunks (E:11158-11257), a launch per group: each does nothing once
    // the scan has stopped
    pend.bufs[0] = work + lm_scratch(M, chunk, rb, false, false).total();
    pend.bufs[1] = static_cast<uint8_t *>(pend.bufs[0]) + part_b;
    qmm::ScanStep last{};
    // At batch 1 with three or more launches' worth of groups, the groups
    // after the first run as one launch (launch_gemv_scan): it applies the
    // first group's step before any weight request (a stop there ends the
    // scan, as the per-group launches would), then reads every later chunk,
    // folding each chunk's best, and its last workgroup to finish decides
    // those chunks in order — the same results with one launch in place of
    // one per later group (the later checkpoints stop nothing in flight).
    const int cf = groups.size() >= 3 ? groups[1].first : ce;  // the folded chunks: [cf, ce)
    const bool fold_shape = M == 1 && groups.size() >= 3 && ce - cf <= qmm::kFoldChunks &&
                            params->chunk_rows % (4 * qmm::kScanRows) == 0;
    for (size_t gi = 0; gi < groups.size(); ++gi) {
        const auto &gr = groups[gi];
        if (gi == 1 && fold_shape && (!pend.on || pend.nparts <= 1024)) {
            qmm_matrix_task tf = tc;
            const int64_t r0 = int64_t(cf) * params->chunk_rows;
            tf.w_base = wb + size_t(r0) * rb;
            tf.rows = int(std::min<int64_t>(int64_t(ce) * params->chunk_rows, vocab_rows) - r0);
            tf.dst_stride = size_t(tf.rows);
            qmm::ScanPlan plan{};
            plan.nch = ce - cf;
            plan.chunk_groups = params->chunk_rows / qmm::kScanRows;
            plan.row_base = uint32_t(r0);
            for (int c = cf; c < ce; ++c) {
                if (params->n_thresholds > 0 && c >= params->first_checkpoint) plan.ckpt |= 1ull << (c - cf);
                plan.thresh[c - cf] = c < params->n_thresholds ? params->thresholds[c] : -1e30f;  // E:11245-11246
            }
            plan.best_val = best_val;
            plan.best_id = best_id;
            plan.st = scan_state;
            plan.c0 = cf;
            qmm::Q8KView xk;
            qmm::Q80View x0;
            act_views(q8k, q80, 1, K, xk, x0);
            qmm::PrevStep pre{};
            if (pend.on)
                pre = qmm::PrevStep{pend.part, pend.nparts, pend.row_base, pend.thresh, pend.checkpoint ? 1 : 0,
                                    pend.c, best_val, best_id, scan_state};
            const qmm::MatArgs af = mat_args(tf, 1, K, scan_state);
            if (qmm::launch_gemv_scan(tf.type, af, xk, pend.x32, pend.gamma, plan, pre, false, ctx->stream) ==
                    hipSuccess &&
                ensure_fold(ctx)) {
                plan.fold = ctx->fold;
                pend.on = false;
                e = qmm::launch_gemv_scan(tf.type, af, xk, pend.x32, pend.gamma, plan, pre, true, ctx->stream);
                return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "scan launch");
            }
        }
        const int c = gr.second;  // the group's last chunk: its threshold and checkpoint
        const int r0 = gr.first * params->chunk_rows;
        qmm_matrix_task t = tc;
        t.w_base = wb + size_t(r0) * rb;
        t.rows = int(std::min<int64_t>(int64_t(c + 1) * params->chunk_rows, vocab_rows) - r0);
        t.dst_stride = size_t(t.rows);
        qmm::ScanStep step;
        step.cand = cand;
        step.draft = draft_ids;
        step.margin = params->prune_margin;
        step.thresh = c < params->n_thresholds ? params->thresholds[c] : -1e30f;  // E:11245-11246
        step.checkpoint = params->n_thresholds > 0 && c >= params->first_checkpoint;
        step.c = c;
        last = step;
        if ((rc = lm_argmax_run(ctx, q8k, q80, M, K, t, uint32_t(r0), nullptr, 0u, nullptr, best_val, best_id, work,
                                scan_state, &step, M == 1 ? &pend : nullptr)))
            return rc;
    }
    return launch_pending(ctx, pend, best_val, best_id, last, scan_state);
}

int qmm_lm_head_scan(qmm_context *ctx, const void *q8k, const void *q80, int M, int K, const void *w_lm,
                     uint32_t type, int vocab_rows, const qmm_lm_scan_params *params, const uint32_t *pre_ids,
                     int n_pre, const uint32_t *draft_ids, float *best_val, uint32_t *best_id, int32_t *scan_state) {
    if (!ctx) return QMM_EINVAL;
    return lm_scan(ctx, q8k, q80, nullptr, nullptr, nullptr, M, K, w_lm, type, vocab_rows, params, pre_ids, n_pre,
                   draft_ids, best_val, best_id, scan_state);
}

int qmm_lm_head_scan_rmsnorm(qmm_context *ctx, const float *x, const float *gamma, int M, int K, const void *w_lm,
                             uint32_t type, int vocab_rows, const qmm_lm_scan_params *params,
                             const uint32_t *pre_ids, int n_pre, const uint32_t *draft_ids, float *best_val,
                             uint32_t *best_id, int32_t *scan_state) {
    if (!ctx) return QMM_EINVAL;
    if (!x || !gamma) return fail(ctx, QMM_EINVAL, "null x or gamma");
    if (M <= 0 || K <= 0) return fail(ctx, QMM_EINVAL, "bad LM-head scan arguments");
    if (K % 256) return fail(ctx, QMM_ESHAPE, "K must be a multiple of 256");
    if (K > 16384) return fail(ctx, QMM_ESHAPE, "K above 16384");
    if (!aligned(x, 16) || !aligned(gamma, 16)) return fail(ctx, QMM_EALIGN, "x and gamma must be 16-B aligned");
    int rc = use_device(ctx);
    if (rc) return rc;
    // the norm's output buffers, for the scans that take the norm's own launch
    const bool q80 = type == QMM_TYPE_Q8_0;
    const size_t k_bytes = qmm::Q8KLayout(M, K).total;
    const size_t y_bytes = q80 ? align256(size_t(M) * size_t(K) * 4) : 0;
    const size_t z_bytes = q80 ? qmm::Q80Layout(M, K).total : 0;
    if ((rc = ensure_act(ctx, k_bytes + y_bytes + z_bytes))) return rc;
    uint8_t *base = static_cast<uint8_t *>(ctx->act);
    return lm_scan(ctx, base, q80 ? base + k_bytes + y_bytes : nullptr, x, gamma,
                   q80 ? reinterpret_cast<float *>(base + k_bytes) : nullptr, M, K, w_lm, type, vocab_rows, params,
                   pre_ids, n_pre, draft_ids, best_val, best_id, scan_state);
}

int qmm_graph_begin(qmm_context *ctx) {
    if (!ctx) return QMM_EINVAL;
    if (ctx->capturing) return fail(ctx, QMM_EINVAL, "capture already active");
    int rc = use_device(ctx);
    if (rc) return rc;
    hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamBeginCapture");
    ctx->capturing = true;
    return QMM_OK;
}

int qmm_graph_end(qmm_context *ctx, void **graph_exec) {
    if (!ctx || !graph_exec) return fail(ctx, QMM_EINVAL, "bad graph_end arguments");
    if (!ctx->capturing) return fail(ctx, QMM_EINVAL, "no capture active");
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
    hipGraphExec_t ex = nullptr;
    e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphInstantiate");
    *graph_exec = ex;
    ++ctx->live_graphs;  // its kernels hold the context's current buffers
    return QMM_OK;
}

int qmm_stream_read(qmm_context *ctx, const void *src, size_t bytes, int workgroups, int loads_per_wave,
                    uint32_t *sink) {
    if (!ctx) return QMM_EINVAL;
    if (!src || !sink || bytes == 0 || workgroups <= 0 || workgroups > (1 << 20))
        return fail(ctx, QMM_EINVAL, "bad stream_read arguments");
    if (!aligned(src, 16) || !aligned(sink, 4)) return fail(ctx, QMM_EALIGN, "src must be 16-B aligned");
    int rc = use_device(ctx);
    if (rc) return rc;
    const hipError_t e = qmm::launch_stream_read(src, bytes, workgroups, loads_per_wave, sink, ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "stream_read launch");
}

int qmm_graph_launch(qmm_context *ctx, void *graph_exec) {
    if (!ctx || !graph_exec) return fail(ctx, QMM_EINVAL, "bad graph_launch arguments");
    hipError_t e = hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "hipGraphLaunch");
}

int qmm_graph_destroy(qmm_context *ctx, void *graph_exec) {
    if (!ctx || !graph_exec) return fail(ctx, QMM_EINVAL, "bad graph_destroy arguments");
    int rc = use_device(ctx);
    if (rc) return rc;
    (void)hipStreamSynchronize(ctx->stream);  // (a replay may still be running)
    const hipError_t e = hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec));
    if (ctx->live_graphs > 0 && --ctx->live_graphs == 0) free_retired(ctx);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "hipGraphExecDestroy");
}

int qmm_timer_begin(qmm_context *ctx) {
    if (!ctx) return QMM_EINVAL;
    hipError_t e = hipEventRecord(ctx->ev0, ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "hipEventRecord");
}

int qmm_timer_end(qmm_context *ctx, float *ms) {
    if (!ctx || !ms) return fail(ctx, QMM_EINVAL, "bad timer_end arguments");
    hipError_t e = hipEventRecord(ctx->ev1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(ctx->ev1);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, ctx->ev0, ctx->ev1);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "hipEventElapsedTime");
}

}  // extern "C"
