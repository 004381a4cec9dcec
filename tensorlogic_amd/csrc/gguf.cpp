// gguf.cpp -- GGUF v2/v3 reader that keeps quantized tensors packed.
//
// Header walk as MmapGGUFLoader::parse_header (src/model/formats/mmap_gguf.rs
// :187-275): magic, version 2..3, tensor/KV counts, KV pairs, tensor infos
// (dims fastest-first in the file, reversed to row-major, gguf.rs:277-291),
// data section aligned.  Differences from the reference, all toward the GGUF
// spec: 1- and 2-byte KV scalars are sized correctly (the reference reads 4
// bytes, mmap_gguf.rs:329-336), general.alignment is honoured (the reference
// fixes 32, :256-257), and every tensor's extent is bounds-checked.
//
// Loading replaces GGUFLoader::load's CPU dequantize-to-f16 (gguf.rs:
// 377-412): Q4_0/Q8_0 bytes go to the device as they are and are repacked
// there; F16 uploads as is; F32 is rounded to F16 on the host (RNE).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>

#include "internal.hpp"

using namespace tlhip;

struct GInfo {
    std::string name;
    uint32_t type = 0;
    int ndim = 0;
    int64_t dims[4] = {1, 1, 1, 1};   // row-major
    uint64_t offset = 0;
    size_t nbytes = 0;
};

struct GKv {
    uint32_t type = 0;
    uint64_t u = 0;
    double f = 0.0;
};

struct tlhip_gguf_s {
    uint8_t* map = nullptr;
    size_t size = 0;
    std::vector<GInfo> infos;
    std::map<std::string, GKv> kv;
    size_t data_off = 0;
};

namespace {

struct Rd {
    const uint8_t* p;
    size_t n, off = 0;
    bool err = false;
    uint64_t u(int bytes) {
        if (off + (size_t)bytes > n) { err = true; return 0; }
        uint64_t v = 0;
        for (int i = 0; i < bytes; i++) v |= (uint64_t)p[off + i] << (8 * i);
        off += bytes;
        return v;
    }
    std::string str() {
        uint64_t len = u(8);
        if (err || len > n - off) { err = true; return {}; }
        std::string s((const char*)p + off, len);
        off += len;
        return s;
    }
};

int scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return -1;
    }
}

bool skip_value(Rd& r, uint32_t t, GKv* out, int depth = 0) {
    if (depth > 4) return false;
    if (t == 8) { r.str(); return !r.err; }
    if (t == 9) {
        uint32_t at = (uint32_t)r.u(4);
        uint64_t n = r.u(8);
        if (r.err) return false;
        for (uint64_t i = 0; i < n; i++)
            if (!skip_value(r, at, nullptr, depth + 1)) return false;
        return true;
    }
    int sz = scalar_size(t);
    if (sz < 0) return false;
    uint64_t v = r.u(sz);
    if (r.err) return false;
    if (out) {
        out->u = v;
        if (t == 6) { uint32_t b = (uint32_t)v; float f; memcpy(&f, &b, 4); out->f = f; }
        else if (t == 12) { double d; memcpy(&d, &v, 8); out->f = d; }
        else if (t == 1) out->f = (double)(int8_t)v;
        else if (t == 3) out->f = (double)(int16_t)v;
        else if (t == 5) out->f = (double)(int32_t)v;
        else if (t == 11) out->f = (double)(int64_t)v;
        else out->f = (double)v;
    }
    return true;
}

size_t type_bytes(uint32_t type, uint64_t nelem, bool* ok) {
    *ok = true;
    switch (type) {
        case 0: return nelem * 4;
        case 1: return nelem * 2;
        case 2: if (nelem % 32) *ok = false; return nelem / 32 * 18;
        case 8: if (nelem % 32) *ok = false; return nelem / 32 * 34;
        case 14: if (nelem % 256) *ok = false; return nelem / 256 * 210;
        default: *ok = false; return 0;
    }
}


}  // namespace

namespace tlhip {

// Round-to-nearest-even f32 -> f16 (host side, for F32 GGUF tensors).
uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return sign;
        uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u, sh = 126u - e;
        uint32_t r = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ax - 0x38000000u;
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}


// Tensor lookup for the model loader: row-major dims, GGUF type id, data.
bool gguf_lookup(tlhip_gguf g, const char* name, uint32_t* type, int* ndim, int64_t dims[4],
                 const uint8_t** data, size_t* nbytes) {
    if (!g || !name) return false;
    for (auto& i : g->infos) {
        if (i.name != name) continue;
        *type = i.type;
        *ndim = i.ndim;
        for (int d = 0; d < 4; d++) dims[d] = i.dims[d];
        *data = g->map + g->data_off + i.offset;
        *nbytes = i.nbytes;
        return true;
    }
    return false;
}

}  // namespace tlhip

extern "C" {

tlhip_status tlhip_gguf_open(const char* path, tlhip_gguf* out) try {
    if (!path || !out) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(TLHIP_ERR_LOAD, "cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return fail(TLHIP_ERR_LOAD, "cannot stat %s", path); }
    size_t size = (size_t)st.st_size;
    if (size < 24) { close(fd); return fail(TLHIP_ERR_LOAD, "%s: file too small for a GGUF header", path); }
    void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return fail(TLHIP_ERR_LOAD, "cannot mmap %s", path);
    auto* g = new tlhip_gguf_s();
    g->map = (uint8_t*)m;
    g->size = size;
    Rd r{g->map, size};
    auto bad = [&](const char* why) {
        tlhip_gguf_close(g);
        return fail(TLHIP_ERR_LOAD, "%s: %s", path, why);
    };
    uint32_t magic = (uint32_t)r.u(4);
    if (magic != 0x46554747u) return bad("invalid GGUF magic");
    uint32_t version = (uint32_t)r.u(4);
    if (version < 2 || version > 3) return bad("unsupported GGUF version (expected 2 or 3)");
    uint64_t nt = r.u(8), nkv = r.u(8);
    if (r.err || nt > (1u << 24) || nkv > (1u << 24)) return bad("corrupt tensor/KV counts");
    // every KV pair takes at least 13 bytes (key length, type, a one-byte
    // value) and every tensor info 32 (name length, rank, one dim, type,
    // offset): counts the file cannot hold are refused before any container
    // is sized by them
    if (nkv * 13 + nt * 32 > size - r.off) return bad("tensor/KV counts exceed the file");
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < nkv; i++) {
        std::string key = r.str();
        uint32_t t = (uint32_t)r.u(4);
        if (r.err) return bad("truncated KV section");
        GKv kv;
        kv.type = t;
        if (!skip_value(r, t, &kv)) return bad("bad KV value");
        if (key == "general.alignment" && t == 4) alignment = kv.u;
        g->kv[key] = kv;
    }
    g->infos.resize(nt);
    for (uint64_t i = 0; i < nt; i++) {
        GInfo& ti = g->infos[i];
        ti.name = r.str();
        uint32_t nd = (uint32_t)r.u(4);
        if (r.err || nd < 1 || nd > 4) return bad("bad tensor rank");
        int64_t raw[4];
        uint64_t nelem = 1;
        for (uint32_t d = 0; d < nd; d++) {
            raw[d] = (int64_t)r.u(8);
            if (raw[d] < 0 || raw[d] > (int64_t)1 << 40) return bad("bad tensor dim");
            // element counts beyond 2^48 cannot fit any file this parser maps;
            // bounding them keeps type_bytes' products (<= 4 * nelem) in range
            if (__builtin_mul_overflow(nelem, (uint64_t)raw[d], &nelem) || nelem > ((uint64_t)1 << 48))
                return bad("tensor element count overflows");
        }
        ti.ndim = (int)nd;
        for (uint32_t d = 0; d < nd; d++) ti.dims[d] = raw[nd - 1 - d];
        ti.type = (uint32_t)r.u(4);
        ti.offset = r.u(8);
        if (r.err) return bad("truncated tensor info");
        bool ok;
        ti.nbytes = type_bytes(ti.type, nelem, &ok);
        if (!ok && (ti.type == 0 || ti.type == 1 || ti.type == 2 || ti.type == 8 || ti.type == 14))
            return bad("tensor size is not a whole number of blocks");
    }
    if (alignment == 0 || (alignment & (alignment - 1))) return bad("bad general.alignment");
    g->data_off = (r.off + alignment - 1) / alignment * alignment;
    if (g->data_off > size) return bad("tensor data exceeds file");
    // each tensor's [offset, offset + nbytes) must lie inside the data section;
    // compared as differences so that no sum can wrap
    const size_t data_bytes = size - g->data_off;
    for (auto& ti : g->infos)
        if (ti.offset > data_bytes || ti.nbytes > data_bytes - ti.offset) return bad("tensor data exceeds file");
    *out = g;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_gguf_close(tlhip_gguf g) try {
    if (!g) return TLHIP_OK;
    if (g->map) munmap(g->map, g->size);
    delete g;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

int tlhip_gguf_n_tensors(tlhip_gguf g) try { return g ? (int)g->infos.size() : 0; } TLHIP_CATCH_VALUE(0)

const char* tlhip_gguf_tensor_name(tlhip_gguf g, int i) try {
    if (!g || i < 0 || i >= (int)g->infos.size()) return nullptr;
    return g->infos[i].name.c_str();
} TLHIP_CATCH_VALUE(nullptr)

tlhip_status tlhip_gguf_kv_u32(tlhip_gguf g, const char* key, uint32_t* v) try {
    if (!g || !key || !v) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(TLHIP_ERR_LOAD, "GGUF key %s not found", key);
    *v = (uint32_t)it->second.u;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_gguf_kv_f32(tlhip_gguf g, const char* key, float* v) try {
    if (!g || !key || !v) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(TLHIP_ERR_LOAD, "GGUF key %s not found", key);
    *v = (float)it->second.f;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_gguf_load_tensor(tlhip_ctx ctx, tlhip_gguf g, const char* name, tlhip_tensor* out) try {
    TLHIP_TRY(check_ctx(ctx));
    if (!g || !name || !out) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const GInfo* ti = nullptr;
    for (auto& i : g->infos)
        if (i.name == name) ti = &i;
    if (!ti) return fail(TLHIP_ERR_LOAD, "tensor %s not found in GGUF", name);
    const uint8_t* src = g->map + g->data_off + ti->offset;
    tlhip_dtype dt;
    switch (ti->type) {
        case 0: case 1: dt = TLHIP_F16; break;
        case 2: dt = TLHIP_Q4_0; break;
        case 8: dt = TLHIP_Q8_0; break;
        case 14: dt = TLHIP_Q6_K; break;
        default: return fail(TLHIP_ERR_DTYPE, "tensor %s: GGUF type %u not supported on the device", name, ti->type);
    }
    if (is_quant(dt) && ti->ndim != 2)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "quantized tensor %s must be 2-D", name);
    tlhip_tensor t;
    TLHIP_TRY(alloc_tensor(ctx, dt, ti->ndim, ti->dims, &t));
    tlhip_status st;
    if (ti->type == 0) {
        size_t n = ti->nbytes / 4;
        std::vector<uint16_t> h(n);
        for (size_t i = 0; i < n; i++) {
            float f;
            memcpy(&f, src + 4 * i, 4);
            h[i] = f32_to_f16(f);
        }
        st = tlhip_tensor_upload(ctx, t, h.data(), n * 2);
    } else {
        st = tlhip_tensor_upload(ctx, t, src, ti->nbytes);
    }
    if (st != TLHIP_OK) {
        tlhip_tensor_free(t);
        return st;
    }
    *out = t;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

}  // extern "C"
