// qmm_gguf.cpp — GGUF v2/v3 container: header, key/value section, tensor
// table, data section (parse_gguf_file E:376-413, find_tensor E:415-420),
// memory-mapped read-only, plus device residency of one tensor's packed
// rows (the reference reads them in place from its mmap, E:4174).
//
// Same rules as the reference: magic "GGUF", version 2 or 3, u64 counts;
// key/value values are skipped by type (scalars, strings, arrays incl.
// string arrays); general.alignment (u32 or u64) overrides the default 32;
// a tensor is name, n_dims (1..4), dims (u64), ggml type, relative offset;
// byte size by compute_ggml_bytes (E:364-374: F32, F16, Q8_0, Q4_K, Q5_K,
// Q6_K; 0 for other types); data starts at the first multiple of the
// alignment after the table. Names are kept to 127 bytes. Unlike the
// reference this parser also checks that every tensor's bytes lie inside
// the file and accepts up to 65536 tensors (the reference stops at 512).
#include "../../include/qmm_hip.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <vector>

struct qmm_gguf {
    int fd = -1;
    const uint8_t *base = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0;
    std::vector<qmm_gguf_tensor> tensors;
};

namespace {

struct Reader {
    const uint8_t *base;
    size_t size, pos = 0;
    bool bytes(void *dst, size_t n) {
        if (n > size - pos) return false;
        memcpy(dst, base + pos, n);
        pos += n;
        return true;
    }
    bool u32(uint32_t &v) { return bytes(&v, 4); }
    bool u64(uint64_t &v) { return bytes(&v, 8); }
    bool skip(uint64_t n) {
        if (n > size - pos) return false;
        pos += size_t(n);
        return true;
    }
    bool str(char *out, size_t cap) {  // keeps at most cap - 1 bytes
        uint64_t len;
        if (!u64(len) || len > size - pos) return false;
        if (out && cap) {
            const size_t c = len < cap - 1 ? size_t(len) : cap - 1;
            memcpy(out, base + pos, c);
            out[c] = '\0';
        }
        pos += size_t(len);
        return true;
    }
};

size_t scalar_size(uint32_t vtype) {  // gguf_scalar_size, E:315-323
    switch (vtype) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}

// parse_or_skip_gguf_value, E:325-361; *val gets u32 / u64 scalars
bool value(Reader &r, uint32_t vtype, uint64_t *val) {
    if (vtype == 8) return r.str(nullptr, 0);
    if (vtype == 9) {
        uint32_t et;
        uint64_t n;
        if (!r.u32(et) || !r.u64(n)) return false;
        if (et == 8) {
            for (uint64_t i = 0; i < n; ++i)
                if (!r.str(nullptr, 0)) return false;
            return true;
        }
        const size_t es = scalar_size(et);
        if (es == 0 || n > (r.size - r.pos) / es) return false;
        return r.skip(n * es);
    }
    const size_t sz = scalar_size(vtype);
    if (sz == 0 || sz > r.size - r.pos) return false;
    if (vtype == 4) {
        uint32_t v;
        memcpy(&v, r.base + r.pos, 4);
        *val = v;
    } else if (vtype == 10) {
        memcpy(val, r.base + r.pos, 8);
    }
    r.pos += sz;
    return true;
}

uint64_t ggml_bytes(uint32_t type, uint64_t n) {  // compute_ggml_bytes, E:364-374
    switch (type) {
        case 0: return n * 4;
        case 1: return n * 2;
        case 8: return n / 32 * 34;
        case 12: return n / 256 * 144;
        case 13: return n / 256 * 176;
        case 14: return n / 256 * 210;
        default: return 0;
    }
}

int parse(qmm_gguf *g) {
    Reader r{g->base, g->size};
    uint8_t magic[4];
    uint64_t nt, nkv;
    if (!r.bytes(magic, 4) || memcmp(magic, "GGUF", 4) != 0) return QMM_EINVAL;
    if (!r.u32(g->version) || g->version < 2 || g->version > 3) return QMM_EINVAL;
    if (!r.u64(nt) || !r.u64(nkv) || nt > 65536) return QMM_EINVAL;
    g->alignment = 32;
    char key[128];
    for (uint64_t i = 0; i < nkv; ++i) {
        uint32_t vt;
        uint64_t v = 0;
        if (!r.str(key, sizeof(key)) || !r.u32(vt) || !value(r, vt, &v)) return QMM_EINVAL;
        if (strcmp(key, "general.alignment") == 0 && v > 0) g->alignment = v;
    }
    g->tensors.resize(size_t(nt));
    for (auto &t : g->tensors) {
        memset(&t, 0, sizeof(t));
        if (!r.str(t.name, sizeof(t.name)) || !r.u32(t.n_dims) || t.n_dims < 1 || t.n_dims > 4) return QMM_EINVAL;
        t.n_elems = 1;
        for (int d = 0; d < 4; ++d) t.dims[d] = 1;
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            if (!r.u64(t.dims[d])) return QMM_EINVAL;
            t.n_elems *= t.dims[d];
        }
        if (!r.u32(t.type) || !r.u64(t.rel_offset)) return QMM_EINVAL;
        t.byte_size = ggml_bytes(t.type, t.n_elems);
    }
    const uint64_t a = g->alignment ? g->alignment : 32;
    g->data_offset = (uint64_t(r.pos) + a - 1) / a * a;
    for (auto &t : g->tensors) {
        t.abs_offset = g->data_offset + t.rel_offset;
        if (t.abs_offset > g->size || t.byte_size > g->size - t.abs_offset) return QMM_ESHAPE;
    }
    return QMM_OK;
}

}  // namespace

extern "C" {

int qmm_gguf_open(const char *path, qmm_gguf **out) {
    if (!path || !out) return QMM_EINVAL;
    *out = nullptr;
    auto *g = new qmm_gguf();
    g->fd = open(path, O_RDONLY);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || st.st_size < 24) {
        if (g->fd >= 0) close(g->fd);
        delete g;
        return QMM_EINVAL;
    }
    g->size = size_t(st.st_size);
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        close(g->fd);
        delete g;
        return QMM_ENOMEM;
    }
    g->base = static_cast<const uint8_t *>(m);
    const int rc = parse(g);
    if (rc != QMM_OK) {
        qmm_gguf_close(g);
        return rc;
    }
    *out = g;
    return QMM_OK;
}

int qmm_gguf_close(qmm_gguf *g) {
    if (!g) return QMM_EINVAL;
    if (g->base) munmap(const_cast<uint8_t *>(g->base), g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
    return QMM_OK;
}

int qmm_gguf_header(const qmm_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset,
                    int *n_tensors) {
    if (!g) return QMM_EINVAL;
    if (version) *version = g->version;
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    if (n_tensors) *n_tensors = int(g->tensors.size());
    return QMM_OK;
}

int qmm_gguf_tensor_at(const qmm_gguf *g, int i, qmm_gguf_tensor *out) {
    if (!g || !out || i < 0 || size_t(i) >= g->tensors.size()) return QMM_EINVAL;
    *out = g->tensors[size_t(i)];
    return QMM_OK;
}

int qmm_gguf_find_tensor(const qmm_gguf *g, const char *name, qmm_gguf_tensor *out) {
    if (!g || !name) return QMM_EINVAL;
    for (const auto &t : g->tensors)
        if (strcmp(t.name, name) == 0) {
            if (out) *out = t;
            return QMM_OK;
        }
    return QMM_ENOTFOUND;
}

const void *qmm_gguf_data(const qmm_gguf *g, const qmm_gguf_tensor *t) {
    if (!g || !t || t->abs_offset > g->size) return nullptr;
    return g->base + t->abs_offset;
}

int qmm_gguf_upload(qmm_context *ctx, const qmm_gguf *g, const char *name, void **dev_blocks,
                    qmm_gguf_tensor *info) {
    if (!ctx || !g || !name || !dev_blocks) return QMM_EINVAL;
    qmm_gguf_tensor t;
    int rc = qmm_gguf_find_tensor(g, name, &t);
    if (rc != QMM_OK) return rc;
    if (info) *info = t;
    // rows = product of dims 1..3, cols = dims[0] (ggml's innermost dimension)
    const int64_t cols = int64_t(t.dims[0]);
    const int64_t rows = int64_t(t.n_elems / (t.dims[0] ? t.dims[0] : 1));
    return qmm_weight_upload(ctx, g->base + t.abs_offset, t.type, rows, cols, dev_blocks);
}

}  // extern "C"
