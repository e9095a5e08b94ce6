/* GGUF v2/v3 reader (host side of the C ABI, include/le_gguf.h).
 *
 * Replaces the reference's Gguf::open (src/gguf.rs:95-122) and the tensor addressing of
 * cpu_ref::Model (src/cpu_ref.rs:56-58 absolute offsets, :70-85 expert slabs of the 3D
 * ffn_*_exps tensors). The file layout is the public GGUF description: magic "GGUF", u32 version,
 * u64 tensor count, u64 kv count, the kv pairs, the tensor infos, padding to general.alignment
 * (default 32), then the tensor data; tensor offsets are relative to the data start. All integers
 * are little-endian. The same plausibility limits as the reference apply (strings up to 2^28
 * bytes, arrays up to 2^30 elements, at most 2^24 tensors and kv pairs, at most 8 dims).
 */
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/le_gguf.h"
#include "../../include/le_qmm.h"
#include "le_formats.h"

namespace {

struct KV {
    int type = 0;         /* GGUF value type 0..12 */
    uint64_t u = 0;       /* unsigned / bool / signed (two's complement) payload */
    double f = 0.0;       /* F32 / F64 */
    std::string s;        /* string */
    int elem_type = -1;   /* arrays: element type and count */
    uint64_t count = 0;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0; /* relative to the data start */
};

struct Reader {
    FILE *f;
    uint64_t pos = 0;
    bool ok = true;
    std::string err;
    bool bytes(void *dst, size_t n) {
        if (!ok) return false;
        if (n && fread(dst, 1, n, f) != n) return fail("truncated file");
        pos += n;
        return true;
    }
    bool fail(const char *m) {
        if (ok) err = m;
        ok = false;
        return false;
    }
    template <class T>
    T num() {
        uint8_t b[sizeof(T)] = {};
        bytes(b, sizeof(T));
        uint64_t v = 0;
        for (size_t i = 0; i < sizeof(T); i++) v |= (uint64_t)b[i] << (8 * i);
        T out;
        memcpy(&out, &v, sizeof(T)); /* little-endian host */
        return out;
    }
    bool str(std::string &s) {
        const uint64_t n = num<uint64_t>();
        if (!ok) return false;
        if (n > (1ull << 28)) return fail("string too long");
        s.resize((size_t)n);
        return bytes(&s[0], (size_t)n);
    }
    /* one value of `type`; arrays keep their element type and count, their elements are read past */
    bool value(int type, KV &kv, int depth) {
        kv.type = type;
        switch (type) {
        case 0: kv.u = num<uint8_t>(); break;
        case 1: kv.u = (uint64_t)(int64_t)num<int8_t>(); break;
        case 2: kv.u = num<uint16_t>(); break;
        case 3: kv.u = (uint64_t)(int64_t)num<int16_t>(); break;
        case 4: kv.u = num<uint32_t>(); break;
        case 5: kv.u = (uint64_t)(int64_t)num<int32_t>(); break;
        case 6: kv.f = num<float>(); break;
        case 7: kv.u = num<uint8_t>() != 0; break;
        case 8: return str(kv.s);
        case 9: {
            if (depth > 8) return fail("arrays nested too deeply");
            const int et = (int)num<uint32_t>();
            const uint64_t n = num<uint64_t>();
            if (!ok) return false;
            if (n > (1ull << 30)) return fail("array too long");
            kv.elem_type = et;
            kv.count = n;
            KV e;
            for (uint64_t i = 0; i < n && ok; i++) {
                if (!value(et, e, depth + 1)) return false;
                if (et == 8) e.s.clear();
            }
            break;
        }
        case 10: kv.u = num<uint64_t>(); break;
        case 11: kv.u = (uint64_t)num<int64_t>(); break;
        case 12: kv.f = num<double>(); break;
        default: return fail("unknown value type");
        }
        return ok;
    }
};

bool is_signed(int t) { return t == 1 || t == 3 || t == 5 || t == 11; }

/* Value::as_u64 (src/gguf.rs:14-22): unsigned types and bool as they are, signed types when >= 0 */
bool as_u64(const KV &v, uint64_t *out) {
    switch (v.type) {
    case 0: case 2: case 4: case 10: case 7: *out = v.u; return true;
    case 1: case 3: case 5: case 11:
        if ((int64_t)v.u < 0) return false;
        *out = v.u;
        return true;
    }
    return false;
}

}  // namespace

struct le_gguf {
    std::string path;
    uint32_t version = 0;
    std::map<std::string, KV> kv;
    std::vector<Tensor> tensors;
    std::map<std::string, int> by_name;
    uint64_t data_start = 0;
    uint64_t file_size = 0;
    std::string err;
};

static thread_local std::string g_open_error;

extern "C" {

int le_gguf_open(const char *path, le_gguf **out) {
    if (!path || !out) return LE_ERR_ARG;
    *out = nullptr;
    FILE *f = fopen(path, "rb");
    if (!f) {
        g_open_error = std::string("cannot open ") + path;
        return LE_ERR_ARG;
    }
    Reader r{f};
    le_gguf *g = new le_gguf();
    g->path = path;
    char magic[4] = {};
    r.bytes(magic, 4);
    if (r.ok && memcmp(magic, "GGUF", 4) != 0) r.fail("not a GGUF file");
    if (r.ok) {
        g->version = r.num<uint32_t>();
        if (r.ok && (g->version < 2 || g->version > 3)) r.fail("unsupported GGUF version");
    }
    uint64_t nt = 0, nkv = 0;
    if (r.ok) {
        nt = r.num<uint64_t>();
        nkv = r.num<uint64_t>();
        if (r.ok && (nt > (1ull << 24) || nkv > (1ull << 24))) r.fail("implausible counts");
    }
    for (uint64_t i = 0; i < nkv && r.ok; i++) {
        std::string k;
        if (!r.str(k)) break;
        const int t = (int)r.num<uint32_t>();
        KV v;
        if (!r.ok || !r.value(t, v, 0)) break;
        g->kv[k] = v; /* a repeated key keeps the last value, as a map insert does */
    }
    for (uint64_t i = 0; i < nt && r.ok; i++) {
        Tensor t;
        if (!r.str(t.name)) break;
        const uint32_t nd = r.num<uint32_t>();
        if (!r.ok) break;
        if (nd > 8) {
            r.fail("too many dims");
            break;
        }
        for (uint32_t d = 0; d < nd; d++) t.dims.push_back(r.num<uint64_t>());
        t.type = r.num<uint32_t>();
        t.offset = r.num<uint64_t>();
        if (!r.ok) break;
        g->by_name[t.name] = (int)g->tensors.size();
        g->tensors.push_back(t);
    }
    if (r.ok) {
        uint64_t align = 32;
        auto it = g->kv.find("general.alignment");
        uint64_t a = 0;
        if (it != g->kv.end() && as_u64(it->second, &a)) align = a;
        if (align < 1) align = 1;
        g->data_start = (r.pos + align - 1) / align * align;
        if (fseeko(f, 0, SEEK_END) == 0) g->file_size = (uint64_t)ftello(f);
    }
    fclose(f);
    if (!r.ok) {
        g_open_error = r.err;
        delete g;
        return LE_ERR_SHAPE;
    }
    *out = g;
    return LE_OK;
}

const char *le_gguf_open_error(void) { return g_open_error.c_str(); }

void le_gguf_close(le_gguf *g) { delete g; }

int le_gguf_version(const le_gguf *g) { return g ? (int)g->version : 0; }
uint64_t le_gguf_data_start(const le_gguf *g) { return g ? g->data_start : 0; }
int le_gguf_tensor_count(const le_gguf *g) { return g ? (int)g->tensors.size() : 0; }
int le_gguf_kv_count(const le_gguf *g) { return g ? (int)g->kv.size() : 0; }

int le_gguf_find(const le_gguf *g, const char *name) {
    if (!g || !name) return -1;
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? -1 : it->second;
}

/* Bytes of tensor t (product of its dims over the block geometry), with every product and the
 * end of its data (data_start + offset + bytes) checked against overflow and the file size.
 * Returns false when the tensor does not fit the file or its type has no block geometry. */
static bool tensor_extent(const le_gguf *g, const Tensor &t, uint64_t *bytes) {
    uint64_t n = 1;
    for (uint64_t d : t.dims)
        if (__builtin_mul_overflow(n, d, &n)) return false;
    int v = 0, b = 0;
    if (!le_block_geometry((int)t.type, &v, &b) || n % (uint64_t)v) return false;
    uint64_t nb = 0, start = 0, end = 0;
    if (__builtin_mul_overflow(n / (uint64_t)v, (uint64_t)b, &nb) || __builtin_add_overflow(g->data_start, t.offset, &start) ||
        __builtin_add_overflow(start, nb, &end) || end > g->file_size)
        return false;
    *bytes = nb;
    return true;
}

int le_gguf_tensor_info(const le_gguf *g, int i, const char **name, int *ggml_type, int *n_dims, uint64_t *dims,
                        uint64_t *offset, uint64_t *nbytes) {
    if (!g || i < 0 || i >= (int)g->tensors.size()) return LE_ERR_ARG;
    const Tensor &t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = (int)t.type;
    if (n_dims) *n_dims = (int)t.dims.size();
    if (dims)
        for (size_t d = 0; d < 8; d++) dims[d] = d < t.dims.size() ? t.dims[d] : 1;
    if (offset) *offset = g->data_start + t.offset;
    /* a type without block geometry reports 0 bytes; a tensor whose size overflows or whose data
     * runs past the end of the file is an error (its name, type and dims are still reported) */
    int v = 0, b = 0;
    uint64_t nb = 0;
    const bool known = le_block_geometry((int)t.type, &v, &b) != 0;
    const bool fits = tensor_extent(g, t, &nb);
    if (nbytes) *nbytes = fits ? nb : 0;
    return !known || fits ? LE_OK : LE_ERR_SHAPE;
}

/* Expert e's slab of a 3D tensor (dims [cols, rows, n_expert]): cpu_ref::expert_parts,
 * src/cpu_ref.rs:70-85. Also valid for 2D tensors with expert 0. */
int le_gguf_expert_slab(const le_gguf *g, const char *name, int expert, uint64_t *offset, uint64_t *bytes) {
    const int i = le_gguf_find(g, name);
    if (i < 0) return LE_ERR_ARG;
    const Tensor &t = g->tensors[(size_t)i];
    int v = 0, b = 0;
    if (!le_block_geometry((int)t.type, &v, &b)) return LE_ERR_TYPE;
    if (t.dims.empty() || t.dims[0] % (uint64_t)v) return LE_ERR_SHAPE;
    const uint64_t rows = t.dims.size() > 1 ? t.dims[1] : 1, nexp = t.dims.size() > 2 ? t.dims[2] : 1;
    if (expert < 0 || (uint64_t)expert >= nexp) return LE_ERR_ARG;
    uint64_t total = 0, slab = 0;
    /* the whole tensor inside the file (overflow-checked), so every slab of it is too */
    if (!tensor_extent(g, t, &total)) return LE_ERR_SHAPE;
    if (__builtin_mul_overflow(t.dims[0] / (uint64_t)v * (uint64_t)b, rows, &slab) || slab > total ||
        (uint64_t)expert * slab + slab > total)
        return LE_ERR_SHAPE;
    if (offset) *offset = g->data_start + t.offset + (uint64_t)expert * slab;
    if (bytes) *bytes = slab;
    return LE_OK;
}

int le_gguf_kv_type(const le_gguf *g, const char *key) {
    if (!g || !key) return -1;
    auto it = g->kv.find(key);
    return it == g->kv.end() ? -1 : it->second.type;
}

int le_gguf_kv_u64(const le_gguf *g, const char *key, uint64_t *out) {
    if (!g || !key || !out) return LE_ERR_ARG;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || !as_u64(it->second, out)) return LE_ERR_TYPE;
    return LE_OK;
}

int le_gguf_kv_i64(const le_gguf *g, const char *key, int64_t *out) {
    if (!g || !key || !out) return LE_ERR_ARG;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return LE_ERR_TYPE;
    const KV &v = it->second;
    if (is_signed(v.type) || v.type == 0 || v.type == 2 || v.type == 4 || v.type == 7 || (v.type == 10 && v.u <= INT64_MAX)) {
        *out = (int64_t)v.u;
        return LE_OK;
    }
    return LE_ERR_TYPE;
}

/* Value::as_f32 (src/gguf.rs:24): F32, or F64 narrowed */
int le_gguf_kv_f32(const le_gguf *g, const char *key, float *out) {
    if (!g || !key || !out) return LE_ERR_ARG;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || (it->second.type != 6 && it->second.type != 12)) return LE_ERR_TYPE;
    *out = (float)it->second.f;
    return LE_OK;
}

int le_gguf_kv_str(const le_gguf *g, const char *key, const char **out) {
    if (!g || !key || !out) return LE_ERR_ARG;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 8) return LE_ERR_TYPE;
    *out = it->second.s.c_str();
    return LE_OK;
}

int le_gguf_kv_array(const le_gguf *g, const char *key, int *elem_type, uint64_t *count) {
    if (!g || !key) return LE_ERR_ARG;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 9) return LE_ERR_TYPE;
    if (elem_type) *elem_type = it->second.elem_type;
    if (count) *count = it->second.count;
    return LE_OK;
}

int le_gguf_read(const le_gguf *g, uint64_t offset, uint64_t bytes, void *dst) {
    if (!g || (!dst && bytes)) return LE_ERR_ARG;
    if (offset > g->file_size || bytes > g->file_size - offset) return LE_ERR_SHAPE;
    FILE *f = fopen(g->path.c_str(), "rb");
    if (!f) return LE_ERR_ARG;
    int rc = LE_OK;
    if (fseeko(f, (off_t)offset, SEEK_SET) != 0 || fread(dst, 1, (size_t)bytes, f) != (size_t)bytes) rc = LE_ERR_SHAPE;
    fclose(f);
    return rc;
}

}  // extern "C"
