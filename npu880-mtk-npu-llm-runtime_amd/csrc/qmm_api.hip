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
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/qmm_hip.h"
#include "qmm_device.h"

struct qmm_context {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    void *act = nullptr;  // Q8_K + Q8_0 activation buffers of the dispatcher
    size_t act_cap = 0;
    void *lm = nullptr;   // LM-head epilogue scratch: logits | argmax slices | gathered rows
    size_t lm_cap = 0;
    bool capturing = false;
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
    return t == qmm::kQ8_0 || t == qmm::kQ4_K || t == qmm::kQ5_K || t == qmm::kQ6_K;
}
int block_values(uint32_t t) { return t == qmm::kQ8_0 ? 32 : 256; }

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int ensure_act(qmm_context *ctx, size_t bytes) {
    if (bytes <= ctx->act_cap) return QMM_OK;
    if (ctx->capturing)
        return fail(ctx, QMM_ENOMEM,
                    "activation buffers too small during graph capture: call qmm_reserve first");
    if (ctx->act) {
        hipError_t e = hipFree(ctx->act);
        ctx->act = nullptr;
        ctx->act_cap = 0;
        if (e != hipSuccess) return hip_fail(ctx, e, "hipFree");
    }
    hipError_t e = hipMalloc(&ctx->act, bytes);
    if (e != hipSuccess) {
        ctx->act = nullptr;
        (void)hipGetLastError();
        return fail(ctx, QMM_ENOMEM, "hipMalloc of activation buffers failed");
    }
    ctx->act_cap = bytes;
    return QMM_OK;
}

int ensure_lm(qmm_context *ctx, size_t bytes) {
    if (bytes <= ctx->lm_cap) return QMM_OK;
    if (ctx->capturing)
        return fail(ctx, QMM_ENOMEM, "LM-head scratch too small during graph capture: run once before capturing");
    if (ctx->lm) {
        (void)hipStreamSynchronize(ctx->stream);
        hipError_t e = hipFree(ctx->lm);
        ctx->lm = nullptr;
        ctx->lm_cap = 0;
        if (e != hipSuccess) return hip_fail(ctx, e, "hipFree");
    }
    hipError_t e = hipMalloc(&ctx->lm, bytes);
    if (e != hipSuccess) {
        ctx->lm = nullptr;
        (void)hipGetLastError();
        return fail(ctx, QMM_ENOMEM, "hipMalloc of LM-head scratch failed");
    }
    ctx->lm_cap = bytes;
    return QMM_OK;
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// the LM-head epilogue: rows of one tensor (contiguous, or gathered by id)
// on prequantized activations, then the running argmax update
int gemv_argmax_fused(qmm_context *ctx, const void *q8k, const void *q80, int K, qmm_matrix_task *t,
                      const uint32_t *ids, uint32_t row_base, bool round16, void *part, float *best_val,
                      uint32_t *best_id, bool *done);

int lm_argmax(qmm_context *ctx, const void *q8k, const void *q80, int M, int K, const void *w, uint32_t type,
              int rows, uint32_t row_base, const uint32_t *ids, float *logits_out, float *best_val,
              uint32_t *best_id) {
    if (!ctx) return QMM_EINVAL;
    if (!w || !best_val || !best_id || M <= 0 || K <= 0 || rows <= 0)
        return fail(ctx, QMM_EINVAL, "bad LM-head arguments");
    if (!supported(type)) return fail(ctx, QMM_ETYPE, "unsupported ggml type");
    if (!aligned(best_val, 4) || !aligned(best_id, 4)) return fail(ctx, QMM_EALIGN, "best_val/best_id must be 4-B aligned");
    const size_t rb = qmm_row_bytes(type, K);
    const size_t logit_b = logits_out ? 0 : align256(size_t(M) * rows * 4);
    // partials: per 1024-row slice, or (M = 1) per workgroup of the fused grid
    const size_t part_b = align256(std::max(qmm::argmax_scratch_bytes(M, rows),
                                            M == 1 ? size_t(qmm::kMaxArgmaxParts) * sizeof(qmm::Best) : size_t(0)));
    const size_t gather_b = ids ? align256(size_t(rows) * rb) : 0;
    int rc = use_device(ctx);
    if (rc) return rc;
    if ((rc = ensure_lm(ctx, logit_b + part_b + gather_b))) return rc;
    uint8_t *scr = static_cast<uint8_t *>(ctx->lm);
    float *logits = logits_out ? logits_out : reinterpret_cast<float *>(scr);
    void *part = scr + logit_b;
    const void *wrows = w;
    if (ids) {
        uint8_t *g = scr + logit_b + part_b;
        hipError_t e = qmm::launch_gather_rows(static_cast<const uint8_t *>(w), rb, ids, rows, g, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "row gather launch");
        wrows = g;
    }
    qmm_matrix_task t{};
    t.w_base = wrows;
    t.type = type;
    t.row_bytes = rb;
    t.dst = logits;
    t.dst_stride = size_t(rows);
    t.residual = nullptr;
    t.res_stride = 0;
    t.rows = rows;
    t.cols = K;
    if (M == 1) {  // the GEMV's persistent grid reduces to one partial per workgroup
        bool done = false;
        rc = gemv_argmax_fused(ctx, q8k, q80, K, &t, ids, row_base, ids == nullptr, part, best_val, best_id, &done);
        if (rc || done) return rc;
    }
    rc = qmm_gemm_multi_dispatch_prequantized(ctx, q8k, q80, M, K, &t, 1);
    if (rc) return rc;
    hipError_t e = qmm::launch_argmax(logits, M, rows, size_t(rows), /*round16=*/ids == nullptr, ids, row_base,
                                      best_val, best_id, part, ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "argmax launch");
}

// Validate the task list against (M, K) and assign start_row.
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
            const uintptr_t wa = (T.type == qmm::kQ4_K || T.type == qmm::kQ5_K) ? 16 : 2;
            if (!aligned(T.w_base, wa)) return fail(ctx, QMM_EALIGN, "task " + std::to_string(t) + ": weight base misaligned for its format");
            if (!aligned(T.dst, 4) || (T.residual && !aligned(T.residual, 4))) return fail(ctx, QMM_EALIGN, "task " + std::to_string(t) + ": dst/residual not 4-B aligned");
        }
        if (M == 1 && qmm::gemv_lds_bytes(T.type, K) > 65536)
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
    xk = {nullptr, nullptr, nullptr, nullptr};
    x0 = {nullptr, nullptr};
    if (q8k) {
        const qmm::Q8KLayout L(M, K);
        const uint8_t *b = static_cast<const uint8_t *>(q8k);
        xk = {reinterpret_cast<const int8_t *>(b), reinterpret_cast<const float *>(b + L.d_off),
              reinterpret_cast<const int32_t *>(b + L.bs_off), reinterpret_cast<const int8_t *>(b + L.tile_off)};
    }
    if (q80) {
        const qmm::Q80Layout L(M, K);
        const uint8_t *b = static_cast<const uint8_t *>(q80);
        x0 = {reinterpret_cast<const int8_t *>(b), reinterpret_cast<const float *>(b + L.d_off)};
    }
}

// x32 != nullptr (M = 1 only): the GEMV kernels quantize x themselves.
int run_tasks(qmm_context *ctx, const float *x32, const void *q8k, const void *q80, int M, int K,
              const qmm_matrix_task *tasks, int n_tasks) {
    qmm::Q8KView xk;
    qmm::Q80View x0;
    act_views(q8k, q80, M, K, xk, x0);
    // tasks of one type run as one launch (up to kMaxGroup per launch), in
    // order of first appearance; outputs are disjoint, so grouping changes
    // no result
    bool done[256] = {};
    for (int t0 = 0; t0 < n_tasks; ++t0) {
        if (done[t0] || tasks[t0].rows == 0) continue;
        qmm::MatArgs group[qmm::kMaxGroup];
        int n = 0;
        for (int t = t0; t < n_tasks; ++t) {
            const qmm_matrix_task &T = tasks[t];
            if (done[t] || T.rows == 0 || T.type != tasks[t0].type) continue;
            done[t] = true;
            qmm::MatArgs &a = group[n++];
            a.w = static_cast<const uint8_t *>(T.w_base);
            a.row_bytes = T.row_bytes;
            a.N = T.rows;
            a.K = K;
            a.M = M;
            a.y = T.dst;
            a.ldy = M > 1 ? T.dst_stride : size_t(T.rows);
            a.res = T.residual;
            a.ldr = M > 1 ? T.res_stride : size_t(T.rows);
            if (n == qmm::kMaxGroup) break;
        }
        const hipError_t e = (M == 1) ? qmm::launch_gemv(tasks[t0].type, group, n, x32, xk, x0, ctx->stream)
                                      : qmm::launch_mfma(tasks[t0].type, group, n, xk, x0, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "matmul launch");
    }
    return QMM_OK;
}

// M = 1 LM head: the prequantized dispatch's checks, then the GEMV with the
// running argmax fused and the final combine. *done stays false (nothing
// launched) where the fused grid does not apply.
int gemv_argmax_fused(qmm_context *ctx, const void *q8k, const void *q80, int K, qmm_matrix_task *t,
                      const uint32_t *ids, uint32_t row_base, bool round16, void *part, float *best_val,
                      uint32_t *best_id, bool *done) {
    *done = false;
    bool need_q8k, need_q80;
    int rc = check_tasks(ctx, 1, K, t, 1, &need_q8k, &need_q80);
    if (rc) return rc;
    if (need_q8k && !q8k) return fail(ctx, QMM_EINVAL, "K-quant task without Q8_K activations");
    if (need_q80 && !q80) return fail(ctx, QMM_EINVAL, "Q8_0 task without Q8_0 activations");
    if ((q8k && !aligned(q8k, 16)) || (q80 && !aligned(q80, 16)))
        return fail(ctx, QMM_EALIGN, "activation buffers must be 16-B aligned");
    qmm::Q8KView xk;  // (the caller has made the context's device current)
    qmm::Q80View x0;
    act_views(need_q8k ? q8k : nullptr, need_q80 ? q80 : nullptr, 1, K, xk, x0);
    qmm::MatArgs a;
    a.w = static_cast<const uint8_t *>(t->w_base);
    a.row_bytes = t->row_bytes;
    a.N = t->rows;
    a.K = K;
    a.M = 1;
    a.y = t->dst;
    a.ldy = size_t(t->rows);
    a.res = nullptr;
    a.ldr = size_t(t->rows);
    int nparts = 0;
    hipError_t e = qmm::launch_gemv_argmax(t->type, a, xk, x0, round16, part, &nparts, ctx->stream);
    if (e == hipErrorNotSupported) return QMM_OK;
    if (e != hipSuccess) return hip_fail(ctx, e, "GEMV + argmax launch");
    e = qmm::launch_argmax_final(part, nparts, ids, row_base, best_val, best_id, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "argmax launch");
    *done = true;
    return QMM_OK;
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
    return ensure_act(ctx, qmm::Q8KLayout(max_M, max_K).total + qmm::Q80Layout(max_M, max_K).total);
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
    const size_t k_bytes = need_q8k ? qmm::Q8KLayout(M, K).total : 0;
    const size_t z_bytes = need_q80 ? qmm::Q80Layout(M, K).total : 0;
    if ((rc = ensure_act(ctx, k_bytes + z_bytes))) return rc;
    void *q8k = need_q8k ? ctx->act : nullptr;
    void *q80 = need_q80 ? static_cast<uint8_t *>(ctx->act) + k_bytes : nullptr;
    hipError_t e;
    if (need_q8k && (e = qmm::launch_quantize_q8k(x, M, K, q8k, ctx->stream)) != hipSuccess)
        return hip_fail(ctx, e, "quantize_q8k launch");
    if (need_q80 && (e = qmm::launch_quantize_q8_0(x, M, K, q80, ctx->stream)) != hipSuccess)
        return hip_fail(ctx, e, "quantize_q8_0 launch");
    return run_tasks(ctx, nullptr, q8k, q80, M, K, tasks, n_tasks);
}

int qmm_gemm_multi_dispatch_prequantized(qmm_context *ctx, const void *q8k, const void *q80, int M,
                                         int K, qmm_matrix_task *tasks, int n_tasks) {
    if (!ctx) return QMM_EINVAL;
    bool need_q8k, need_q80;
    int rc = check_tasks(ctx, M, K, tasks, n_tasks, &need_q8k, &need_q80);
    if (rc) return rc;
    if (need_q8k && !q8k) return fail(ctx, QMM_EINVAL, "K-quant task without Q8_K activations");
    if (need_q80 && !q80) return fail(ctx, QMM_EINVAL, "Q8_0 task without Q8_0 activations");
    if ((q8k && !aligned(q8k, 16)) || (q80 && !aligned(q80, 16)))
        return fail(ctx, QMM_EALIGN, "activation buffers must be 16-B aligned");
    if ((rc = use_device(ctx))) return rc;
    return run_tasks(ctx, nullptr, need_q8k ? q8k : nullptr, need_q80 ? q80 : nullptr, M, K, tasks,
                     n_tasks);
}

int qmm_lm_head_argmax(qmm_context *ctx, const void *q8k, const void *q80, int M, int K, const void *w_rows,
                       uint32_t type, int rows, uint32_t row_base, float *logits_out, float *best_val,
                       uint32_t *best_id) {
    return lm_argmax(ctx, q8k, q80, M, K, w_rows, type, rows, row_base, nullptr, logits_out, best_val, best_id);
}

int qmm_eval_rows_argmax(qmm_context *ctx, const void *q8k, const void *q80, int M, int K, const void *w_tensor,
                         uint32_t type, const uint32_t *row_ids, int n_ids, float *vals_out, float *best_val,
                         uint32_t *best_id) {
    if (ctx && !row_ids) return fail(ctx, QMM_EINVAL, "row_ids is NULL");
    return lm_argmax(ctx, q8k, q80, M, K, w_tensor, type, n_ids, 0, row_ids, vals_out, best_val, best_id);
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
    return QMM_OK;
}

int qmm_graph_launch(qmm_context *ctx, void *graph_exec) {
    if (!ctx || !graph_exec) return fail(ctx, QMM_EINVAL, "bad graph_launch arguments");
    hipError_t e = hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), ctx->stream);
    return e == hipSuccess ? QMM_OK : hip_fail(ctx, e, "hipGraphLaunch");
}

int qmm_graph_destroy(void *graph_exec) {
    if (!graph_exec) return QMM_EINVAL;
    return hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)) == hipSuccess ? QMM_OK : QMM_EHIP;
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
