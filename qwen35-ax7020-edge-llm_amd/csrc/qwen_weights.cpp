// qwen_weights.cpp -- the weight-image loader: reads the exporter's manifest
// and converts every BFP8 tensor of the image to the GPU layout once
// (C ABI in include/qwen_kernels.h).
//
// Image format (05/export_qwen35_weights_bfp8_64k.py:64-80, :159-174): tensors
// at 64-byte aligned file offsets; a "block64_bfp8" tensor of shape [M, K] is
// its mantissa plane (int8 [M][K], row-major 64-element blocks) followed by
// its exponent plane (one byte per block, padded to a multiple of 8 with 127,
// 05/bfp8_packer.py:53-86); "raw_fp32" and "raw_bf16" tensors are plain
// little-endian arrays.  The engine slices a BFP8 tensor as mant = raw[:M*K],
// exps = raw[M*K : M*K + M*K/64] (04/qwen_real_engine.py:834-846); the
// converted planes are cached under exactly those host addresses, so later
// bfp8_gemv / forward calls on the engine's pointers find them resident.
#include <hip/hip_runtime.h>

#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "host_internal.h"

namespace qhost {
namespace {

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) ---------------------
struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    double num = 0.0;
    bool b = false;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal* get(const char* key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonReader {
  public:
    JsonReader(const char* p, size_t n) : p_(p), end_(p + n) {}
    bool parse(JVal* out) {
        if (!value(out, 0)) return false;
        ws();
        return p_ == end_;
    }
    size_t offset(const char* base) const { return (size_t)(p_ - base); }

  private:
    const char* p_;
    const char* end_;
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* s) {
        const size_t n = strlen(s);
        if ((size_t)(end_ - p_) < n || memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    bool string(std::string* out) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        out->clear();
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c != '\\') {
                out->push_back(c);
                continue;
            }
            if (p_ >= end_) return false;
            c = *p_++;
            switch (c) {
                case '"': case '\\': case '/': out->push_back(c); break;
                case 'b': out->push_back('\b'); break;
                case 'f': out->push_back('\f'); break;
                case 'n': out->push_back('\n'); break;
                case 'r': out->push_back('\r'); break;
                case 't': out->push_back('\t'); break;
                case 'u': {
                    if (end_ - p_ < 4) return false;
                    unsigned cp = 0;
                    for (int i = 0; i < 4; ++i) {
                        const char h = *p_++;
                        cp <<= 4;
                        if (h >= '0' && h <= '9') cp |= (unsigned)(h - '0');
                        else if (h >= 'a' && h <= 'f') cp |= (unsigned)(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') cp |= (unsigned)(h - 'A' + 10);
                        else return false;
                    }
                    // UTF-8 of a BMP code point (tensor names are ASCII)
                    if (cp < 0x80) {
                        out->push_back((char)cp);
                    } else if (cp < 0x800) {
                        out->push_back((char)(0xC0 | (cp >> 6)));
                        out->push_back((char)(0x80 | (cp & 0x3F)));
                    } else {
                        out->push_back((char)(0xE0 | (cp >> 12)));
                        out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
                        out->push_back((char)(0x80 | (cp & 0x3F)));
                    }
                    break;
                }
                default: return false;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool value(JVal* v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v->kind = JVal::Obj;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                ws();
                std::pair<std::string, JVal> kv;
                if (!string(&kv.first)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                if (!value(&kv.second, depth + 1)) return false;
                v->obj.push_back(std::move(kv));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            v->kind = JVal::Arr;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                JVal e;
                if (!value(&e, depth + 1)) return false;
                v->arr.push_back(std::move(e));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            v->kind = JVal::Str;
            return string(&v->str);
        }
        if (lit("true")) {
            v->kind = JVal::Bool;
            v->b = true;
            return true;
        }
        if (lit("false")) {
            v->kind = JVal::Bool;
            return true;
        }
        if (lit("null")) return true;
        // number
        std::string num;
        while (p_ < end_ && (strchr("+-0123456789.eE", *p_) != nullptr)) num.push_back(*p_++);
        if (num.empty()) return false;
        char* e = nullptr;
        errno = 0;
        v->num = strtod(num.c_str(), &e);
        v->kind = JVal::Num;
        return e && *e == '\0' && errno == 0;
    }
};

// ---- manifest entries ------------------------------------------------------------------------------
enum { T_BFP8 = 0, T_F32 = 1, T_BF16 = 2 };

struct Entry {
    std::string name;
    int type = -1;
    std::vector<int64_t> shape;
    uint64_t offset = 0, bytes = 0, mant_bytes = 0, exp_bytes = 0;
};

bool as_u64(const JVal* v, uint64_t* out) {
    if (!v || v->kind != JVal::Num || v->num < 0 || v->num > 9.0e15 || v->num != (double)(uint64_t)v->num)
        return false;
    *out = (uint64_t)v->num;
    return true;
}

// Parses the manifest and checks every tensor against the exporter's rules.
int read_manifest(const char* path, size_t image_bytes, std::vector<Entry>* out) {
    FILE* f = fopen(path, "rb");
    if (!f) {
        set_error("manifest %s: %s", path, strerror(errno));
        return BFP8_EINVAL;
    }
    std::string text;
    char buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
    fclose(f);
    JVal root;
    JsonReader rd(text.data(), text.size());
    if (!rd.parse(&root) || root.kind != JVal::Obj) {
        set_error("manifest %s: not valid JSON (near byte %zu)", path, rd.offset(text.data()));
        return BFP8_EINVAL;
    }
    const JVal* tensors = root.get("tensors");
    if (!tensors || tensors->kind != JVal::Obj) {
        set_error("manifest %s: no \"tensors\" object", path);
        return BFP8_EINVAL;
    }
    for (const auto& kv : tensors->obj) {
        Entry e;
        e.name = kv.first;
        const JVal& t = kv.second;
        const JVal* type = t.get("type");
        const JVal* shape = t.get("shape");
        if (t.kind != JVal::Obj || !type || type->kind != JVal::Str || !shape || shape->kind != JVal::Arr ||
            !as_u64(t.get("file_offset"), &e.offset) || !as_u64(t.get("byte_size"), &e.bytes)) {
            set_error("manifest: tensor %s lacks type, shape, file_offset or byte_size", e.name.c_str());
            return BFP8_EINVAL;
        }
        uint64_t count = 1;
        for (const JVal& d : shape->arr) {
            uint64_t v;
            if (!as_u64(&d, &v)) {
                set_error("manifest: tensor %s has a bad shape", e.name.c_str());
                return BFP8_EINVAL;
            }
            e.shape.push_back((int64_t)v);
            count *= v;
        }
        if (type->str == "block64_bfp8") {
            e.type = T_BFP8;
            if (!as_u64(t.get("mantissa_bytes"), &e.mant_bytes) || !as_u64(t.get("exponent_bytes"), &e.exp_bytes)) {
                set_error("manifest: BFP8 tensor %s lacks mantissa_bytes / exponent_bytes", e.name.c_str());
                return BFP8_EINVAL;
            }
            const uint64_t blocks = count / 64;
            if (e.shape.size() != 2 || e.shape[1] % 64 != 0 || e.shape[0] <= 0 || e.shape[0] > INT32_MAX ||
                e.shape[1] > INT32_MAX || e.mant_bytes != count || e.exp_bytes != (blocks + 7) / 8 * 8 ||
                e.bytes != e.mant_bytes + e.exp_bytes) {
                set_error("manifest: BFP8 tensor %s is not [M, K] with K %% 64 == 0, M*K mantissa bytes and "
                          "ceil8(M*K/64) exponent bytes", e.name.c_str());
                return BFP8_EINVAL;
            }
        } else if (type->str == "raw_fp32" || type->str == "raw_bf16") {
            e.type = type->str == "raw_fp32" ? T_F32 : T_BF16;
            if (e.bytes != count * (e.type == T_F32 ? 4u : 2u)) {
                set_error("manifest: tensor %s: byte_size does not match its shape", e.name.c_str());
                return BFP8_EINVAL;
            }
        } else {
            set_error("manifest: tensor %s has unknown type %s", e.name.c_str(), type->str.c_str());
            return BFP8_EINVAL;
        }
        if (e.offset % 64 != 0 || e.offset > image_bytes || e.bytes > image_bytes - e.offset) {
            set_error("manifest: tensor %s [%llu, +%llu) is unaligned or outside the %zu-byte image", e.name.c_str(),
                      (unsigned long long)e.offset, (unsigned long long)e.bytes, image_bytes);
            return BFP8_EINVAL;
        }
        out->push_back(std::move(e));
    }
    return BFP8_OK;
}

struct Loaded {
    const int8_t* mant;
    const uint8_t* exps;
    int M, K;
};
std::map<std::string, Loaded> g_loaded;  // by manifest name (g.mu held)

}  // namespace

void weights_index_clear() { g_loaded.clear(); }

}  // namespace qhost

using namespace qhost;

extern "C" {

int qwen_weights_scan(const char* manifest_json, size_t image_bytes, int* n_bfp8, int* n_f32, int* n_bf16,
                      uint64_t* bfp8_bytes) {
    if (!manifest_json) return BFP8_EINVAL;
    std::vector<Entry> es;
    int rc = read_manifest(manifest_json, image_bytes, &es);
    if (rc) return rc;
    int c[3] = {0, 0, 0};
    uint64_t wb = 0;
    for (const Entry& e : es) {
        ++c[e.type];
        if (e.type == T_BFP8) wb += e.bytes;
    }
    if (n_bfp8) *n_bfp8 = c[T_BFP8];
    if (n_f32) *n_f32 = c[T_F32];
    if (n_bf16) *n_bf16 = c[T_BF16];
    if (bfp8_bytes) *bfp8_bytes = wb;
    return (int)es.size();
}

int qwen_weights_preload(const void* image, size_t image_bytes, const char* manifest_json) {
    if (!image || !manifest_json) return BFP8_EINVAL;
    std::vector<Entry> es;
    int rc = read_manifest(manifest_json, image_bytes, &es);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g.mu);
    if ((rc = ensure_init_locked())) return rc;
    const uint8_t* base = static_cast<const uint8_t*>(image);
    int n = 0;
    for (const Entry& e : es) {
        const uint8_t* p = base + e.offset;
        if (e.type == T_BFP8) {
            const int M = (int)e.shape[0], K = (int)e.shape[1];
            const int8_t* mant = reinterpret_cast<const int8_t*>(p);
            const uint8_t* exps = p + (size_t)M * K;
            DevWeights w;
            if ((rc = weights_cached(mant, exps, M, K, true, &w))) return rc;
            g_loaded[e.name] = Loaded{reinterpret_cast<const int8_t*>(w.mant), w.exps, M, K};
            ++n;
        } else if (e.type == T_BF16 && e.shape.size() == 2 && e.shape[0] <= INT32_MAX && e.shape[1] <= INT32_MAX) {
            const uint16_t* d;
            int tiled;
            if ((rc = bf16_table_cached(reinterpret_cast<const uint16_t*>(p), (int)e.shape[0], (int)e.shape[1], true,
                                        &d, &tiled)))
                return rc;
        } else if (e.type == T_F32) {
            if ((rc = forward_preload_param(p, e.bytes))) return rc;
        }
    }
    if (hipStreamSynchronize(g.stream) != hipSuccess) {
        set_error("weight conversion failed");
        return BFP8_EHIP;
    }
    return n;
}

int qwen_weights_find(const char* name, const int8_t** mant_gpu, const uint8_t** exps_gpu, int* M, int* K) {
    if (!name) return BFP8_EINVAL;
    std::lock_guard<std::mutex> lk(g.mu);
    auto it = g_loaded.find(name);
    if (it == g_loaded.end()) {
        set_error("qwen_weights_find: %s was not preloaded", name);
        return BFP8_EINVAL;
    }
    if (mant_gpu) *mant_gpu = it->second.mant;
    if (exps_gpu) *exps_gpu = it->second.exps;
    if (M) *M = it->second.M;
    if (K) *K = it->second.K;
    return BFP8_OK;
}

int bfp8_dev_pack_rows(int8_t* mant_gpu, uint8_t* exps_gpu, const uint8_t* row_stream, int M, int K, void* stream) {
    if (M < 0 || K < 0 || (K & 63) || (M > 0 && K > 0 && (!mant_gpu || !exps_gpu || !row_stream))) return BFP8_EINVAL;
    {
        std::lock_guard<std::mutex> lk(g.mu);
        if (ensure_init_locked() != BFP8_OK) return BFP8_EHIP;
    }
    const size_t nb = (size_t)(K >> 6), stride = nb + (size_t)K;
    HIP_OK(bfp8_launch_pack_strided(reinterpret_cast<uint8_t*>(mant_gpu), exps_gpu,
                                    reinterpret_cast<const int8_t*>(row_stream + nb), stride, row_stream, stride, M, K,
                                    pick_stream(stream)));
    return BFP8_OK;
}

}  // extern "C"
