// GGUF files into the buffer type: the parse that ggml's gguf_init_from_file(no_alloc = true) does for
// speech.cpp's ModelFile::open (src/common/model-file.cpp:35-47), and the read of ModelFile::load (:251-268): each
// tensor's bytes from the file in 16 MB pieces, each piece set on the device at its offset.
//
// The format, from the GGUF specification (version 2 and 3; all integers little endian):
//   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv,
//   n_kv x { string key, u32 value type, value },            string = u64 length + bytes (no terminator)
//   n_tensors x { string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset },
//   padding to `general.alignment` (u32 key, default 32), then the data section; a tensor's offset counts from its
//   start and is a multiple of the alignment.
// Value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array {u32 type, u64 n, n values},
// 10 u64, 11 i64, 12 f64.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "../../include/mx.h"
#include "mx_error.h"

struct mx_gguf {
    std::string path;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_offset = 0;
    uint64_t file_size = 0;
    struct Kv {
        std::string key;
        int type = 0;             // value type
        int elem_type = -1;       // arrays: element type
        uint64_t n = 0;           // arrays: element count
        std::vector<uint8_t> raw;  // scalars: the value's bytes; numeric arrays: the elements; strings: the text
        std::vector<std::string> strs;  // arrays of strings
    };
    std::vector<Kv> kvs;
    struct Tensor {
        std::string name;
        int type = 0;
        int n_dims = 0;
        int64_t ne[4] = {1, 1, 1, 1};
        uint64_t offset = 0, nbytes = 0;
    };
    std::vector<Tensor> tensors;
};

namespace {

constexpr size_t kReadPiece = (size_t)16 << 20;  // bytes read from the file and set on the device at a time

// Block geometry of ggml's types (ggml-common.h): elements per block, bytes per block; {0, 0} for types this reader
// does not know.
struct Geo {
    int64_t blck;
    uint64_t bytes;
};
Geo geometry(int type) {
    switch (type) {
        case 0: return {1, 4};      // F32
        case 1: return {1, 2};      // F16
        case 2: return {32, 18};    // Q4_0
        case 3: return {32, 20};    // Q4_1
        case 6: return {32, 22};    // Q5_0
        case 7: return {32, 24};    // Q5_1
        case 8: return {32, 34};    // Q8_0
        case 9: return {32, 36};    // Q8_1
        case 10: return {256, 84};  // Q2_K
        case 11: return {256, 110}; // Q3_K
        case 12: return {256, 144}; // Q4_K
        case 13: return {256, 176}; // Q5_K
        case 14: return {256, 210}; // Q6_K
        case 15: return {256, 292}; // Q8_K
        case 24: return {1, 1};     // I8
        case 25: return {1, 2};     // I16
        case 26: return {1, 4};     // I32
        case 27: return {1, 8};     // I64
        case 28: return {1, 8};     // F64
        case 30: return {1, 2};     // BF16
        default: return {0, 0};
    }
}

uint64_t scalar_size(int vt) {
    switch (vt) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;  // string, array: variable
    }
}

// Sequential reads with the file's remaining size as the bound of every length field.
struct Reader {
    FILE *f;
    uint64_t size, pos = 0;
    std::string why;
    bool get(void *dst, uint64_t n) {
        if (n > size - pos) {
            why = "the file ends inside its header";
            return false;
        }
        if (n && std::fread(dst, 1, (size_t)n, f) != n) {
            why = "a read failed";
            return false;
        }
        pos += n;
        return true;
    }
    template <typename T>
    bool num(T &v) { return get(&v, sizeof v); }
    bool str(std::string &s) {
        uint64_t n;
        if (!num(n)) return false;
        if (n > size - pos) {
            why = "a string runs past the end of the file";
            return false;
        }
        s.resize((size_t)n);
        return get(s.data(), n);
    }
};

bool read_value(Reader &r, mx_gguf::Kv &kv) {
    if (kv.type == 8) {
        std::string s;
        if (!r.str(s)) return false;
        kv.raw.assign(s.begin(), s.end());
        return true;
    }
    if (kv.type == 9) {
        uint32_t et;
        if (!r.num(et) || !r.num(kv.n)) return false;
        kv.elem_type = (int)et;
        if (et == 8) {
            if (kv.n > (r.size - r.pos) / 8) {  // every string takes at least its 8-byte length
                r.why = "an array runs past the end of the file";
                return false;
            }
            kv.strs.resize((size_t)kv.n);
            for (auto &s : kv.strs)
                if (!r.str(s)) return false;
            return true;
        }
        const uint64_t es = scalar_size((int)et);
        if (es == 0) {
            r.why = "an array of arrays or of an unknown type";
            return false;
        }
        if (kv.n > (r.size - r.pos) / es) {
            r.why = "an array runs past the end of the file";
            return false;
        }
        kv.raw.resize((size_t)(kv.n * es));
        return r.get(kv.raw.data(), kv.n * es);
    }
    const uint64_t es = scalar_size(kv.type);
    if (es == 0) {
        r.why = "a value of unknown type " + std::to_string(kv.type);
        return false;
    }
    kv.raw.resize((size_t)es);
    return r.get(kv.raw.data(), es);
}

bool parse(FILE *f, mx_gguf &g, std::string &why) {
    Reader r{f, g.file_size, 0, {}};
    uint32_t magic;
    uint64_t n_tensors, n_kv;
    if (!r.num(magic) || magic != 0x46554747u) {  // "GGUF"
        why = "it does not start with GGUF";
        return false;
    }
    if (!r.num(g.version) || (g.version != 2 && g.version != 3)) {
        why = "its GGUF version is " + std::to_string(g.version) + ", not 2 or 3";
        return false;
    }
    if (!r.num(n_tensors) || !r.num(n_kv)) {
        why = r.why;
        return false;
    }
    // every key-value takes at least 12 bytes and every tensor info 24: counts beyond that are corrupt
    if (n_kv > g.file_size / 12 || n_tensors > g.file_size / 24) {
        why = "its counts of keys and tensors exceed what the file can hold";
        return false;
    }
    g.kvs.resize((size_t)n_kv);
    for (auto &kv : g.kvs) {
        uint32_t vt;
        if (!r.str(kv.key) || !r.num(vt)) {
            why = r.why;
            return false;
        }
        kv.type = (int)vt;
        if (!read_value(r, kv)) {
            why = r.why + " (key " + kv.key + ")";
            return false;
        }
        if (kv.key == "general.alignment") {
            uint32_t a = 0;
            if (kv.type != 4 || (std::memcpy(&a, kv.raw.data(), 4), a == 0) || (a & (a - 1))) {
                why = "general.alignment is not a power of two held as u32";
                return false;
            }
            g.alignment = a;
        }
    }
    g.tensors.resize((size_t)n_tensors);
    for (auto &t : g.tensors) {
        uint32_t nd, type;
        if (!r.str(t.name) || !r.num(nd)) {
            why = r.why;
            return false;
        }
        if (nd < 1 || nd > 4) {
            why = "the tensor " + t.name + " has " + std::to_string(nd) + " dimensions";
            return false;
        }
        t.n_dims = (int)nd;
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t v;
            if (!r.num(v)) {
                why = r.why;
                return false;
            }
            if (v > ((uint64_t)1 << 40)) {
                why = "the tensor " + t.name + " has an axis beyond 2^40";
                return false;
            }
            t.ne[d] = (int64_t)v;
        }
        if (!r.num(type) || !r.num(t.offset)) {
            why = r.why;
            return false;
        }
        t.type = (int)type;
        const Geo geo = geometry(t.type);
        if (geo.blck == 0) {
            why = "the tensor " + t.name + " has the ggml type " + std::to_string(type) + ", which this reader does not know";
            return false;
        }
        if (t.ne[0] % geo.blck != 0) {
            why = "the rows of " + t.name + " are not whole blocks of its type";
            return false;
        }
        // ggml_nbytes of a contiguous tensor; every multiply is checked, so no shape can wrap past the size check
        // (four axes of up to 2^40 would overflow even 128 bits)
        uint64_t n = 0;
        bool wrapped = __builtin_mul_overflow((uint64_t)(t.ne[0] / geo.blck), (uint64_t)geo.bytes, &n);
        for (int d = 1; d < 4 && !wrapped; d++) wrapped = __builtin_mul_overflow(n, (uint64_t)t.ne[d], &n);
        if (wrapped || n > g.file_size) {
            why = "the tensor " + t.name + " is larger than the file";
            return false;
        }
        t.nbytes = n;
        if (t.offset % g.alignment != 0) {
            why = "the tensor " + t.name + " is not aligned to general.alignment";
            return false;
        }
    }
    g.data_offset = (r.pos + g.alignment - 1) / g.alignment * g.alignment;
    for (const auto &t : g.tensors) {
        if (t.offset > g.file_size || t.nbytes > g.file_size - t.offset ||
            g.data_offset > g.file_size - t.offset - t.nbytes) {
            why = "the data of " + t.name + " lies past the end of the file";
            return false;
        }
    }
    return true;
}

bool seek(FILE *f, uint64_t at) { return fseeko(f, (off_t)at, SEEK_SET) == 0; }

}  // namespace

extern "C" {

MX_API mx_gguf *mx_gguf_open(const char *path) {
    if (!path) {
        mx::set_error(MX_INVALID, "null path");
        return nullptr;
    }
    std::unique_ptr<FILE, int (*)(FILE *)> f(std::fopen(path, "rb"), &std::fclose);
    if (!f) {
        mx::set_error(MX_FAILED, (std::string("cannot open ") + path + "; check the path and that the file can be read").c_str());
        return nullptr;
    }
    auto g = std::make_unique<mx_gguf>();
    g->path = path;
    if (fseeko(f.get(), 0, SEEK_END) != 0) {
        mx::set_error(MX_FAILED, (std::string("cannot seek in ") + path).c_str());
        return nullptr;
    }
    g->file_size = (uint64_t)ftello(f.get());
    std::rewind(f.get());
    std::string why;
    bool ok = false;
    try {
        ok = parse(f.get(), *g, why);
    } catch (const std::bad_alloc &) {  // the bounds keep every container within the file's size; this is the rest
        mx::set_error(MX_ALLOC_FAILED, (std::string("out of host memory reading ") + path).c_str());
        return nullptr;
    }
    if (!ok) {
        mx::set_error(MX_INVALID, (std::string("cannot read ") + path + " as a GGUF file: " + why).c_str());
        return nullptr;
    }
    return g.release();
}

MX_API void mx_gguf_close(mx_gguf *f) { delete f; }

MX_API int64_t mx_gguf_n_tensors(const mx_gguf *f) { return f ? (int64_t)f->tensors.size() : -1; }

MX_API uint64_t mx_gguf_data_offset(const mx_gguf *f) { return f ? f->data_offset : 0; }

MX_API int mx_gguf_get_tensor(const mx_gguf *f, int64_t i, mx_gguf_tensor_info *out) {
    if (!f || !out || i < 0 || i >= (int64_t)f->tensors.size()) return mx::set_error(MX_INVALID, "no such tensor");
    const auto &t = f->tensors[(size_t)i];
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) out->ne[d] = t.ne[d];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    return MX_SUCCESS;
}

MX_API int64_t mx_gguf_find_tensor(const mx_gguf *f, const char *name) {
    if (!f || !name) return -1;
    for (size_t i = 0; i < f->tensors.size(); i++)
        if (f->tensors[i].name == name) return (int64_t)i;
    return -1;
}

MX_API int64_t mx_gguf_n_keys(const mx_gguf *f) { return f ? (int64_t)f->kvs.size() : -1; }

MX_API const char *mx_gguf_key(const mx_gguf *f, int64_t id) {
    return f && id >= 0 && id < (int64_t)f->kvs.size() ? f->kvs[(size_t)id].key.c_str() : nullptr;
}

MX_API int64_t mx_gguf_find_key(const mx_gguf *f, const char *key) {
    if (!f || !key) return -1;
    for (size_t i = 0; i < f->kvs.size(); i++)
        if (f->kvs[i].key == key) return (int64_t)i;
    return -1;
}

MX_API int mx_gguf_key_type(const mx_gguf *f, int64_t id) {
    return f && id >= 0 && id < (int64_t)f->kvs.size() ? f->kvs[(size_t)id].type : -1;
}

MX_API int mx_gguf_get_str(const mx_gguf *f, int64_t id, const char **out, size_t *len) {
    if (!f || id < 0 || id >= (int64_t)f->kvs.size() || !out) return mx::set_error(MX_INVALID, "no such key");
    const auto &kv = f->kvs[(size_t)id];
    if (kv.type != 8) return mx::set_error(MX_INVALID, ("the key " + kv.key + " is not a string").c_str());
    *out = (const char *)kv.raw.data();
    if (len) *len = kv.raw.size();
    return MX_SUCCESS;
}

MX_API int mx_gguf_get_int(const mx_gguf *f, int64_t id, int64_t *out) {
    if (!f || id < 0 || id >= (int64_t)f->kvs.size() || !out) return mx::set_error(MX_INVALID, "no such key");
    const auto &kv = f->kvs[(size_t)id];
    const uint8_t *p = kv.raw.data();
    switch (kv.type) {
        case 0: *out = *p; break;
        case 1: *out = (int8_t)*p; break;
        case 7: *out = *p != 0; break;
        case 2: { uint16_t v; std::memcpy(&v, p, 2); *out = v; break; }
        case 3: { int16_t v; std::memcpy(&v, p, 2); *out = v; break; }
        case 4: { uint32_t v; std::memcpy(&v, p, 4); *out = v; break; }
        case 5: { int32_t v; std::memcpy(&v, p, 4); *out = v; break; }
        case 10: {
            uint64_t v;
            std::memcpy(&v, p, 8);
            if (v > (uint64_t)INT64_MAX) return mx::set_error(MX_INVALID, ("the key " + kv.key + " exceeds int64").c_str());
            *out = (int64_t)v;
            break;
        }
        case 11: std::memcpy(out, p, 8); break;
        default: return mx::set_error(MX_INVALID, ("the key " + kv.key + " is not an integer").c_str());
    }
    return MX_SUCCESS;
}

MX_API int mx_gguf_get_float(const mx_gguf *f, int64_t id, double *out) {
    if (!f || id < 0 || id >= (int64_t)f->kvs.size() || !out) return mx::set_error(MX_INVALID, "no such key");
    const auto &kv = f->kvs[(size_t)id];
    if (kv.type == 6) {
        float v;
        std::memcpy(&v, kv.raw.data(), 4);
        *out = v;
    } else if (kv.type == 12) {
        std::memcpy(out, kv.raw.data(), 8);
    } else {
        return mx::set_error(MX_INVALID, ("the key " + kv.key + " is not a float").c_str());
    }
    return MX_SUCCESS;
}

MX_API int mx_gguf_get_arr(const mx_gguf *f, int64_t id, int *elem_type, uint64_t *n, const void **data) {
    if (!f || id < 0 || id >= (int64_t)f->kvs.size() || !elem_type || !n || !data)
        return mx::set_error(MX_INVALID, "no such key");
    const auto &kv = f->kvs[(size_t)id];
    if (kv.type != 9) return mx::set_error(MX_INVALID, ("the key " + kv.key + " is not an array").c_str());
    *elem_type = kv.elem_type;
    *n = kv.n;
    *data = kv.elem_type == 8 ? nullptr : (const void *)kv.raw.data();
    return MX_SUCCESS;
}

MX_API int mx_gguf_get_arr_str(const mx_gguf *f, int64_t id, uint64_t i, const char **out, size_t *len) {
    if (!f || id < 0 || id >= (int64_t)f->kvs.size() || !out) return mx::set_error(MX_INVALID, "no such key");
    const auto &kv = f->kvs[(size_t)id];
    if (kv.type != 9 || kv.elem_type != 8 || i >= kv.n)
        return mx::set_error(MX_INVALID, ("no string " + std::to_string(i) + " in the key " + kv.key).c_str());
    *out = kv.strs[(size_t)i].c_str();
    if (len) *len = kv.strs[(size_t)i].size();
    return MX_SUCCESS;
}

MX_API int mx_gguf_load_tensor(mx_backend *be, const mx_gguf *f, int64_t i, const mx_tensor *dst) {
    if (!f || i < 0 || i >= (int64_t)f->tensors.size()) return mx::set_error(MX_INVALID, "no such tensor");
    const auto &t = f->tensors[(size_t)i];
    if (!dst || dst->type != t.type) return mx::set_error(MX_INVALID, ("the tensor " + t.name + " is of another type").c_str());
    for (int d = 0; d < 4; d++)
        if (dst->ne[d] != t.ne[d])
            return mx::set_error(MX_INVALID, ("the tensor " + t.name + " has another shape").c_str());
    std::unique_ptr<FILE, int (*)(FILE *)> fp(std::fopen(f->path.c_str(), "rb"), &std::fclose);
    if (!fp) return mx::set_error(MX_FAILED, ("cannot open " + f->path).c_str());
    // the tensor's bytes stream through one host buffer of at most kReadPiece bytes, each piece set at its offset
    std::vector<uint8_t> buf((size_t)std::min<uint64_t>(kReadPiece, t.nbytes));
    uint64_t got = 0;
    if (seek(fp.get(), f->data_offset + t.offset)) {
        while (got < t.nbytes) {
            const size_t want = (size_t)std::min<uint64_t>(buf.size(), t.nbytes - got);
            if (std::fread(buf.data(), 1, want, fp.get()) != want) break;
            const int rc = mx_tensor_set(be, dst, buf.data(), (size_t)got, want);
            if (rc != MX_SUCCESS) return rc;  // its message stands
            got += want;
        }
    }
    if (got < t.nbytes)
        return mx::set_error(MX_FAILED, (f->path + ": tensor " + t.name + " ends past the end of the file (" +
                                         std::to_string(got) + " of its " + std::to_string(t.nbytes) +
                                         " bytes read)").c_str());
    return MX_SUCCESS;
}

}  // extern "C"
