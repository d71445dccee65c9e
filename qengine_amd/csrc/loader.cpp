// On-disk weights: .safetensors files (memory-mapped, header parsed here) and the loader of a quantized matrix from
// compressed-tensors tensors into the W4 / Q8 device layouts.
//
// A .safetensors file is an 8-byte little-endian header length, a JSON object
//   {"<name>": {"dtype": "I32", "shape": [n, k], "data_offsets": [begin, end]}, ..., "__metadata__": {...}}
// and the tensor bytes (offsets relative to the end of the header). The reference reads them the same way
// (src/safetensors.{h,cpp}: mmap + an index by name); its page-cache management is not part of this path.
//
// load_w4 follows the reference's Worker::load_w4 (src/model.cpp:994-1059): the matrix is the concatenation of row
// ranges of one or more tensors <name>.weight_packed (int32 words of 8 nibbles or 4 bytes) and <name>.weight_scale
// (16-bit per 128-k group), sliced to the columns [c0, c1); the bits per weight follow from the packed width and
// the scale width (4: the W4 layout, 8: Q8); GLU matrices ([gate rows][up rows]) are interleaved per 16-row tile
// before the repack.
#include "qe_api.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace {

// ---- a JSON reader for safetensors headers: objects, arrays, strings, integers, true / false / null ----
struct Json {
    enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
    long long num = 0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const std::string& key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonParser {
public:
    JsonParser(const char* p, size_t n, const std::string& what) : p_(p), begin_(p), end_(p + n), what_(what) {}
    Json parse() {
        Json v = value(0);
        ws();
        CHECK(p_ == end_, "%s: trailing bytes after the JSON header", what_.c_str());
        return v;
    }

private:
    const char* p_;
    const char* begin_;
    const char* end_;
    std::string what_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) p_++;
    }
    char peek() {
        ws();
        CHECK(p_ < end_, "%s: JSON header ends early", what_.c_str());
        return *p_;
    }
    void expect(char c) {
        CHECK(peek() == c, "%s: JSON header: expected '%c' at byte %ld", what_.c_str(), c, (long)(p_ - begin_));
        p_++;
    }
    std::string string() {
        expect('"');
        std::string s;
        while (true) {
            CHECK(p_ < end_, "%s: JSON header: unterminated string", what_.c_str());
            const char c = *p_++;
            if (c == '"') break;
            if (c != '\\') {
                s += c;
                continue;
            }
            CHECK(p_ < end_, "%s: JSON header: bad escape", what_.c_str());
            const char e = *p_++;
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {  // code point (BMP) as UTF-8; tensor names are ASCII in practice
                    CHECK(end_ - p_ >= 4, "%s: JSON header: bad \\u escape", what_.c_str());
                    unsigned cp = 0;
                    for (int i = 0; i < 4; i++) {
                        const char h = *p_++;
                        cp = cp * 16 + (h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10
                                        : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99);
                        CHECK(cp < 0x10000, "%s: JSON header: bad \\u escape", what_.c_str());
                    }
                    if (cp < 0x80) s += (char)cp;
                    else if (cp < 0x800) { s += (char)(0xC0 | (cp >> 6)); s += (char)(0x80 | (cp & 63)); }
                    else { s += (char)(0xE0 | (cp >> 12)); s += (char)(0x80 | ((cp >> 6) & 63)); s += (char)(0x80 | (cp & 63)); }
                    break;
                }
                default: CHECK(false, "%s: JSON header: bad escape \\%c", what_.c_str(), e);
            }
        }
        return s;
    }
    Json value(int depth) {
        CHECK(depth < 16, "%s: JSON header nested too deeply", what_.c_str());
        Json v;
        const char c = peek();
        if (c == '{') {
            v.kind = Json::kObj;
            p_++;
            if (peek() == '}') { p_++; return v; }
            while (true) {
                std::string k = string();
                expect(':');
                v.obj.emplace_back(std::move(k), value(depth + 1));
                if (peek() == ',') { p_++; continue; }
                expect('}');
                return v;
            }
        }
        if (c == '[') {
            v.kind = Json::kArr;
            p_++;
            if (peek() == ']') { p_++; return v; }
            while (true) {
                v.arr.push_back(value(depth + 1));
                if (peek() == ',') { p_++; continue; }
                expect(']');
                return v;
            }
        }
        if (c == '"') {
            v.kind = Json::kStr;
            v.str = string();
            return v;
        }
        if (c == '-' || (c >= '0' && c <= '9')) {
            v.kind = Json::kNum;
            bool neg = *p_ == '-';
            if (neg) p_++;
            CHECK(p_ < end_ && *p_ >= '0' && *p_ <= '9', "%s: JSON header: bad number", what_.c_str());
            unsigned long long x = 0;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
                CHECK(x < (1ull << 59), "%s: JSON header: number out of range", what_.c_str());
                x = x * 10 + (unsigned)(*p_++ - '0');
            }
            // fractions / exponents appear only in metadata values, which are strings in safetensors; reject them
            CHECK(p_ == end_ || (*p_ != '.' && *p_ != 'e' && *p_ != 'E'), "%s: JSON header: non-integer number",
                  what_.c_str());
            v.num = neg ? -(long long)x : (long long)x;
            return v;
        }
        auto word = [&](const char* w) {
            const size_t n = strlen(w);
            if ((size_t)(end_ - p_) >= n && memcmp(p_, w, n) == 0) { p_ += n; return true; }
            return false;
        };
        if (word("true")) { v.kind = Json::kBool; v.num = 1; return v; }
        if (word("false")) { v.kind = Json::kBool; return v; }
        if (word("null")) return v;
        CHECK(false, "%s: JSON header: unexpected '%c'", what_.c_str(), c);
        return v;
    }
};

size_t dtype_size(const std::string& d) {
    if (d == "F64" || d == "I64" || d == "U64") return 8;
    if (d == "F32" || d == "I32" || d == "U32") return 4;
    if (d == "F16" || d == "BF16" || d == "I16" || d == "U16") return 2;
    if (d == "I8" || d == "U8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    return 0;
}

}  // namespace

// ---- one mapped file ----
struct StTensor {
    std::string dtype;
    std::vector<long long> shape;
    const char* data = nullptr;
    size_t nbytes = 0;
};

struct StFile {
    std::string path;
    void* map = nullptr;
    size_t size = 0;
    std::map<std::string, StTensor> tensors;
    std::vector<std::string> names;  // sorted (the map's order)

    explicit StFile(const std::string& p) : path(p) {
        const int fd = ::open(p.c_str(), O_RDONLY);
        CHECK(fd >= 0, "safetensors: cannot open %s", p.c_str());
        struct stat sb;
        CHECK(fstat(fd, &sb) == 0, "safetensors: cannot stat %s", p.c_str());
        size = (size_t)sb.st_size;
        CHECK(size >= 8, "safetensors: %s: %zu bytes (no header)", p.c_str(), size);
        map = mmap(nullptr, size, PROT_READ, MAP_SHARED, fd, 0);
        ::close(fd);
        CHECK(map != MAP_FAILED, "safetensors: cannot map %s", p.c_str());
        const char* base = reinterpret_cast<const char*>(map);
        uint64_t hl = 0;
        memcpy(&hl, base, 8);  // little-endian (every target of this library)
        CHECK(hl >= 2 && hl <= size - 8, "safetensors: %s: header length %llu of a %zu-byte file", p.c_str(),
              (unsigned long long)hl, size);
        const Json h = JsonParser(base + 8, (size_t)hl, p).parse();
        CHECK(h.kind == Json::kObj, "safetensors: %s: the header is not an object", p.c_str());
        const char* data0 = base + 8 + hl;
        const size_t dsize = size - 8 - hl;
        for (const auto& kv : h.obj) {
            if (kv.first == "__metadata__") continue;
            const Json& t = kv.second;
            const Json* dt = t.get("dtype");
            const Json* sh = t.get("shape");
            const Json* off = t.get("data_offsets");
            CHECK(t.kind == Json::kObj && dt && dt->kind == Json::kStr && sh && sh->kind == Json::kArr && off &&
                      off->kind == Json::kArr && off->arr.size() == 2,
                  "safetensors: %s: malformed entry %s", p.c_str(), kv.first.c_str());
            StTensor st;
            st.dtype = dt->str;
            const size_t es = dtype_size(st.dtype);
            CHECK(es > 0, "safetensors: %s: %s has the unknown dtype %s", p.c_str(), kv.first.c_str(), st.dtype.c_str());
            // element count and byte size without wrap-around: a header whose dims multiply past 64 bits (e.g.
            // [2^36, 2^32]) must not pass as a small tensor
            size_t count = 1, nbytes = 0;
            for (const Json& d : sh->arr) {
                CHECK(d.kind == Json::kNum && d.num >= 0 && d.num < (1ll << 40), "safetensors: %s: %s: bad shape",
                      p.c_str(), kv.first.c_str());
                st.shape.push_back(d.num);
                CHECK(!__builtin_mul_overflow(count, (size_t)d.num, &count), "safetensors: %s: %s: the shape overflows",
                      p.c_str(), kv.first.c_str());
            }
            CHECK(!__builtin_mul_overflow(count, es, &nbytes), "safetensors: %s: %s: the byte size overflows", p.c_str(),
                  kv.first.c_str());
            // (e - b) == nbytes and e <= dsize: the tensor's bytes lie inside the file's data
            const long long b = off->arr[0].num, e = off->arr[1].num;
            CHECK(off->arr[0].kind == Json::kNum && off->arr[1].kind == Json::kNum && b >= 0 && e >= b &&
                      (size_t)e <= dsize && (size_t)(e - b) == nbytes,
                  "safetensors: %s: %s: data_offsets [%lld, %lld] for %zu elements of %zu bytes (data %zu bytes)",
                  p.c_str(), kv.first.c_str(), b, e, count, es, dsize);
            st.data = data0 + b;
            st.nbytes = (size_t)(e - b);
            CHECK(tensors.emplace(kv.first, std::move(st)).second, "safetensors: %s: duplicate tensor %s", p.c_str(),
                  kv.first.c_str());
        }
        for (const auto& kv : tensors) names.push_back(kv.first);
    }
    ~StFile() {
        if (map && map != MAP_FAILED) munmap(map, size);
    }
    const StTensor* find(const std::string& n) const {
        const auto it = tensors.find(n);
        return it == tensors.end() ? nullptr : &it->second;
    }
    const StTensor& get(const std::string& n) const {
        const StTensor* t = find(n);
        CHECK(t != nullptr, "safetensors: %s has no tensor %s", path.c_str(), n.c_str());
        return *t;
    }
};

// ---- the quantized matrix of row ranges of compressed-tensors tensors ----
struct W4LoadDims {
    int n = 0, k = 0, bits = 0, sdt = kScaleBF16;
};

W4LoadDims w4_load_dims(const StFile& f, const char* const* names, const int* r0, const int* r1, int nspec, int c0,
                        int c1) {
    CHECK(nspec >= 1, "load_w4: no row ranges");
    W4LoadDims d;
    const StTensor& q0 = f.get(std::string(names[0]) + ".weight_packed");
    const StTensor& s0 = f.get(std::string(names[0]) + ".weight_scale");
    CHECK(q0.shape.size() == 2 && s0.shape.size() == 2 && q0.dtype == "I32" &&
              (s0.dtype == "BF16" || s0.dtype == "F16"),
          "load_w4: %s: packed I32 [n][words] and 16-bit scales [n][k/128] expected (%s, %s)", names[0],
          q0.dtype.c_str(), s0.dtype.c_str());
    const long long K = s0.shape[1] * 128;
    CHECK(K > 0 && K < (1ll << 31) && (q0.shape[1] * 32) % K == 0, "load_w4: %s: packed width %lld for K %lld",
          names[0], q0.shape[1], K);
    d.bits = (int)(q0.shape[1] * 32 / K);
    CHECK((d.bits == 4 || d.bits == 8) && q0.shape[1] * 32 == K * d.bits, "load_w4: %s: packed width %lld for K %lld",
          names[0], q0.shape[1], K);
    d.sdt = s0.dtype == "F16" ? kScaleF16 : kScaleBF16;
    CHECK(d.bits == 4 || d.sdt == kScaleBF16, "load_w4: %s: 8-bit matrices take bf16 scales", names[0]);
    if (c0 < 0) {
        c0 = 0;
        c1 = (int)K;
    }
    CHECK(c0 >= 0 && c1 <= K && c0 < c1 && c0 % 128 == 0 && (c1 - c0) % 128 == 0, "load_w4: %s: columns [%d, %d) of %lld",
          names[0], c0, c1, K);
    d.k = c1 - c0;
    long long n = 0;
    for (int i = 0; i < nspec; i++) {
        const StTensor& q = f.get(std::string(names[i]) + ".weight_packed");
        const StTensor& s = f.get(std::string(names[i]) + ".weight_scale");
        CHECK(q.dtype == q0.dtype && s.dtype == s0.dtype && q.shape.size() == 2 && s.shape.size() == 2 &&
                  q.shape[1] == q0.shape[1] && s.shape[1] == s0.shape[1] && q.shape[0] == s.shape[0],
              "load_w4: %s: K / bits / dtype differ from %s", names[i], names[0]);
        CHECK(r0[i] >= 0 && r0[i] < r1[i] && r1[i] <= q.shape[0], "load_w4: %s: rows [%d, %d) of %lld", names[i], r0[i],
              r1[i], q.shape[0]);
        n += r1[i] - r0[i];
    }
    CHECK(n % 16 == 0 && n < (1ll << 30), "load_w4: %lld rows (a multiple of 16)", n);
    d.n = (int)n;
    return d;
}

void w4_load(const StFile& f, const char* const* names, const int* r0, const int* r1, int nspec, int c0, int c1,
             bool glu, void* dq, void* ds, hipStream_t st) {
    const W4LoadDims d = w4_load_dims(f, names, r0, r1, nspec, c0, c1);
    CHECK(!glu || d.n % 32 == 0, "load_w4: GLU needs a multiple of 32 rows (n %d)", d.n);
    if (c0 < 0) c0 = 0;
    const long long K = f.get(std::string(names[0]) + ".weight_scale").shape[1] * 128;
    const size_t rowb = (size_t)d.k * d.bits / 8, srow = (size_t)K * d.bits / 8;  // bytes per row: slice / source
    const size_t sg = (size_t)(d.k / 128), sgs = (size_t)(K / 128);                // scale groups: slice / source
    int32_t* tq = nullptr;
    uint16_t* ts = nullptr;
    HIP_CHECK(hipMalloc(&tq, (size_t)d.n * rowb));
    HIP_CHECK(hipMalloc(&ts, (size_t)d.n * sg * 2));
    int off = 0;
    for (int i = 0; i < nspec; i++) {
        const StTensor& q = f.get(std::string(names[i]) + ".weight_packed");
        const StTensor& s = f.get(std::string(names[i]) + ".weight_scale");
        const int h = r1[i] - r0[i];
        HIP_CHECK(hipMemcpy2DAsync(reinterpret_cast<char*>(tq) + (size_t)off * rowb, rowb,
                                   q.data + (size_t)r0[i] * srow + (size_t)c0 * d.bits / 8, srow, rowb, h,
                                   hipMemcpyHostToDevice, st));
        HIP_CHECK(hipMemcpy2DAsync(ts + (size_t)off * sg, sg * 2, s.data + ((size_t)r0[i] * sgs + c0 / 128) * 2,
                                   sgs * 2, sg * 2, h, hipMemcpyHostToDevice, st));
        off += h;
    }
    int32_t* gq = tq;
    uint16_t* gs = ts;
    if (glu) {
        HIP_CHECK(hipMalloc(&gq, (size_t)d.n * rowb));
        HIP_CHECK(hipMalloc(&gs, (size_t)d.n * sg * 2));
        glu_interleave_rows(tq, ts, d.n, d.k, gq, gs, st, d.bits);
    }
    if (d.bits == 8) repack_q8(gq, gs, d.n, d.k, reinterpret_cast<uint4*>(dq), reinterpret_cast<uint16_t*>(ds), st);
    else repack_w4(gq, gs, d.n, d.k, reinterpret_cast<uint4*>(dq), reinterpret_cast<uint16_t*>(ds), st);
    HIP_CHECK(hipStreamSynchronize(st));
    if (glu) {
        HIP_CHECK(hipFree(gq));
        HIP_CHECK(hipFree(gs));
    }
    HIP_CHECK(hipFree(tq));
    HIP_CHECK(hipFree(ts));
}

// ---- C-ABI ----
extern "C" {

void* qe_st_open(const char* path) {
    CHECK(path != nullptr, "qe_st_open: NULL path");
    return new StFile(path);
}

void qe_st_close(void* st) { delete reinterpret_cast<StFile*>(st); }

int qe_st_count(void* st) { return (int)reinterpret_cast<StFile*>(st)->names.size(); }

const char* qe_st_name(void* st, int i) {
    const StFile* f = reinterpret_cast<StFile*>(st);
    CHECK(i >= 0 && i < (int)f->names.size(), "qe_st_name: index %d of %zu", i, f->names.size());
    return f->names[i].c_str();
}

int qe_st_tensor(void* st, const char* name, char* dtype, int64_t* shape, int* ndim, const void** data,
                 size_t* nbytes) {
    const StTensor* t = reinterpret_cast<StFile*>(st)->find(name);
    if (t == nullptr) return 0;
    if (dtype) {
        strncpy(dtype, t->dtype.c_str(), 11);
        dtype[11] = 0;
    }
    if (ndim) *ndim = (int)t->shape.size();
    if (shape)
        for (size_t i = 0; i < t->shape.size() && i < 8; i++) shape[i] = t->shape[i];
    if (data) *data = t->data;
    if (nbytes) *nbytes = t->nbytes;
    return 1;
}

void qe_load_w4_dims(void* st, const char* const* names, const int* r0, const int* r1, int nspec, int c0, int c1,
                     int* n, int* k, int* bits, int* sdt) {
    const W4LoadDims d = w4_load_dims(*reinterpret_cast<StFile*>(st), names, r0, r1, nspec, c0, c1);
    if (n) *n = d.n;
    if (k) *k = d.k;
    if (bits) *bits = d.bits;
    if (sdt) *sdt = d.sdt;
}

void qe_load_w4(void* st, const char* const* names, const int* r0, const int* r1, int nspec, int c0, int c1, int glu,
                void* dq, void* ds, void* stream) {
    w4_load(*reinterpret_cast<StFile*>(st), names, r0, r1, nspec, c0, c1, glu != 0, dq, ds,
            reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
