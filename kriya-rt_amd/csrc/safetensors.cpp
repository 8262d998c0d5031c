// safetensors.cpp — checkpoint archives for the Q4_G64 path (include/kriya_loader.h).
//
// Host code: a safetensors reader (8-byte little-endian header length, a JSON
// header of {name: {dtype, shape, data_offsets}}, then the data section), files
// mapped read-only, single-file or sharded through model.safetensors.index.json,
// and the binding of Q4 projections into the planar device layout.
// Reference: crates/kriya-core/src/safetensors_loader.rs:18-208 (reader, sharded
// loader), :221-273 and :310-318 (MLX triplet repack, f16 scales), tensor.rs:62-101
// (storage sizes), :266-275 and :373-405 (descriptor and bounds checks);
// crates/kriya-backend-metal/src/encoder.rs:306-418 (require_norm_tensor,
// require_q4_weight), :452-591 (validate_production_checkpoint), :651-703
// (bind_q4_buffer).  The planar triplet is the MLX layout itself, so Path B is
// a copy (plus an f16 -> bf16 pass on the device) rather than a repack.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <unordered_set>
#include <utility>
#include <vector>

#include "kriya_loader.h"
#include "kriya_q4.h"

namespace kr {
int set_error(int code, const char *msg);  // kr_api.hip: the thread-local message of kr_last_error()
}

namespace {

int err(int code, const char *fmt, ...) {
    char buf[768];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return kr::set_error(code, buf);
}
int ok() { return kr::set_error(KR_OK, ""); }

constexpr uint64_t kMaxHeaderBytes = 100ull * 1024 * 1024;  // safetensors_loader.rs:18

// ---------------------------------------------------------------- a small JSON reader
// Enough for safetensors headers and index files: objects, arrays, strings (with
// escapes), numbers (non-negative integers kept exactly), true / false / null.
struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool is_uint = false;  // a non-negative integer that fits in 64 bits
    uint64_t u = 0;
    std::string s;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal *get(const char *key) const {
        for (const auto &kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JParser {
  public:
    JParser(const char *p, size_t n) : p_(p), e_(p + n) {}
    bool parse(JVal &v, std::string &why) {
        depth_ = 0;
        if (!value(v)) {
            why = why_;
            return false;
        }
        ws();
        if (p_ != e_) {
            why = "trailing bytes after the JSON value";
            return false;
        }
        return true;
    }

  private:
    const char *p_, *e_;
    int depth_ = 0;
    std::string why_;
    bool fail(const char *m) {
        why_ = m;
        return false;
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char *w) {
        const size_t n = strlen(w);
        if ((size_t)(e_ - p_) < n || memcmp(p_, w, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void utf8(uint32_t cp, std::string &out) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t &v) {
        if (e_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool str(std::string &out) {
        if (p_ >= e_ || *p_ != '"') return fail("expected a string");
        ++p_;
        while (p_ < e_ && *p_ != '"') {
            const unsigned char c = (unsigned char)*p_++;
            if (c < 0x20) return fail("control character in a string");
            if (c != '\\') {
                out += (char)c;
                continue;
            }
            if (p_ >= e_) return fail("unterminated escape");
            const char x = *p_++;
            switch (x) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return fail("bad \\u escape");
                    if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                        uint32_t lo;
                        if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail("lone low surrogate");
                    }
                    utf8(cp, out);
                    break;
                }
                default: return fail("unknown escape");
            }
        }
        if (p_ >= e_) return fail("unterminated string");
        ++p_;
        return true;
    }
    bool num(JVal &v) {
        bool neg = false, frac = false;
        if (p_ < e_ && *p_ == '-') {
            neg = true;
            ++p_;
        }
        if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad number");
        uint64_t u = 0;
        bool fits = true;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = (uint64_t)(*p_++ - '0');
            if (u > (UINT64_MAX - d) / 10) fits = false;
            u = u * 10 + d;
        }
        if (p_ < e_ && *p_ == '.') {
            frac = true;
            ++p_;
            if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad fraction");
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
            frac = true;
            ++p_;
            if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad exponent");
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        v.kind = JVal::Num;
        v.is_uint = !neg && !frac && fits;
        v.u = v.is_uint ? u : 0;
        return true;
    }
    bool value(JVal &v) {
        if (++depth_ > 64) return fail("nesting deeper than 64");
        ws();
        if (p_ >= e_) return fail("unexpected end");
        bool r = true;
        switch (*p_) {
            case '{': {
                ++p_;
                v.kind = JVal::Obj;
                ws();
                if (p_ < e_ && *p_ == '}') {
                    ++p_;
                    break;
                }
                // Duplicate keys are rejected through a hash set of the object's keys: linear in the key count
                // (a header or weight map names up to ~10^5 tensors).
                std::unordered_set<std::string> seen;
                for (;;) {
                    ws();
                    std::string key;
                    if (!str(key)) return false;
                    ws();
                    if (p_ >= e_ || *p_ != ':') return fail("expected ':'");
                    ++p_;
                    JVal child;
                    if (!value(child)) return false;
                    if (!seen.insert(key).second) return fail("duplicate key in an object");
                    v.obj.emplace_back(std::move(key), std::move(child));
                    ws();
                    if (p_ < e_ && *p_ == ',') {
                        ++p_;
                        continue;
                    }
                    if (p_ < e_ && *p_ == '}') {
                        ++p_;
                        break;
                    }
                    return fail("expected ',' or '}'");
                }
                break;
            }
            case '[': {
                ++p_;
                v.kind = JVal::Arr;
                ws();
                if (p_ < e_ && *p_ == ']') {
                    ++p_;
                    break;
                }
                for (;;) {
                    JVal child;
                    if (!value(child)) return false;
                    v.arr.push_back(std::move(child));
                    ws();
                    if (p_ < e_ && *p_ == ',') {
                        ++p_;
                        continue;
                    }
                    if (p_ < e_ && *p_ == ']') {
                        ++p_;
                        break;
                    }
                    return fail("expected ',' or ']'");
                }
                break;
            }
            case '"':
                v.kind = JVal::Str;
                r = str(v.s);
                break;
            case 't':
                v.kind = JVal::Bool;
                r = lit("true") || fail("bad literal");
                break;
            case 'f':
                v.kind = JVal::Bool;
                r = lit("false") || fail("bad literal");
                break;
            case 'n':
                v.kind = JVal::Null;
                r = lit("null") || fail("bad literal");
                break;
            default: r = num(v);
        }
        --depth_;
        return r;
    }
};

// ---------------------------------------------------------------- dtypes and storage sizes

struct DTypeInfo {
    const char *name;
    int code;
    uint64_t block_elems, block_bytes;
};
// DType::from_safetensors_str (safetensors_loader.rs:36-55); storage per block (tensor.rs:62-101)
const DTypeInfo kDTypes[] = {
    {"F32", KR_ST_F32, 1, 4},        {"F16", KR_ST_F16, 1, 2},     {"BF16", KR_ST_BF16, 1, 2},
    {"F8_E4M3", KR_ST_F8_E4M3, 1, 1}, {"Q4_G64", KR_ST_Q4_G64, 64, 36}, {"Q2_G128", KR_ST_Q2_G128, 128, 36},
    {"Q3_G64", KR_ST_Q3_G64, 64, 28}, {"U32", KR_ST_U32, 1, 4},     {"U8", KR_ST_U8, 1, 1},
    {"I32", KR_ST_I32, 1, 4},        {"I8", KR_ST_I8, 1, 1},
};
const DTypeInfo *dtype_by_name(const std::string &s) {
    for (const auto &d : kDTypes)
        if (s == d.name) return &d;
    return nullptr;
}
const DTypeInfo *dtype_by_code(int c) {
    for (const auto &d : kDTypes)
        if (c == d.code) return &d;
    return nullptr;
}
bool is_float(int c) { return c == KR_ST_BF16 || c == KR_ST_F16 || c == KR_ST_F32; }

// bf16 RNE of an f32 (quantizer.rs:19-24) and f16 -> f32 (quantizer.rs:31-57)
uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = sign;
        } else {  // subnormal: normalise
            int ex = -1;
            uint32_t mm = m;
            do {
                ++ex;
                mm <<= 1;
            } while ((mm & 0x400) == 0);
            u = sign | ((uint32_t)(127 - 15 - ex) << 23) | ((mm & 0x3FF) << 13);
        }
    } else if (e == 0x1F) {
        u = sign | 0x7F800000u | (m << 13);
    } else {
        u = sign | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// ---------------------------------------------------------------- archives

struct Shard {
    std::string name;
    void *map = nullptr;
    size_t size = 0;
    uint64_t data_off = 0;
};

struct Tensor {
    int dtype = 0;
    std::vector<uint64_t> shape;
    uint64_t off = 0, len = 0;  // inside the shard's data section
    int shard = 0;
};

struct Header {
    std::map<std::string, Tensor> tensors;
};

void unmap(Shard &s) {
    if (s.map && s.size) munmap(s.map, s.size);
    s.map = nullptr;
}

int map_file(const std::string &path, Shard &s) {
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return err(KR_E_IO, "cannot open '%s': %s", path.c_str(), strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        close(fd);
        return err(KR_E_IO, "'%s' is not a regular file", path.c_str());
    }
    s.size = (size_t)st.st_size;
    if (s.size < 8) {
        close(fd);
        return err(KR_E_FORMAT, "'%s' is %zu bytes, shorter than the 8-byte header length", path.c_str(), s.size);
    }
    void *m = mmap(nullptr, s.size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return err(KR_E_IO, "cannot map '%s': %s", path.c_str(), strerror(errno));
    s.map = m;
    return KR_OK;
}

// open_safetensors_file (safetensors_loader.rs:67-119) + MappedWeightArchive::open (tensor.rs:373-405)
int parse_header(const std::string &path, Shard &s, int shard_index, Header &h) {
    if (int rc = map_file(path, s)) return rc;
    const uint8_t *b = (const uint8_t *)s.map;
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | b[i];
    if (hlen == 0 || hlen > kMaxHeaderBytes)
        return err(KR_E_FORMAT, "'%s': header length %llu is not in 1..%llu", path.c_str(), (unsigned long long)hlen,
                   (unsigned long long)kMaxHeaderBytes);
    if (8 + hlen > s.size)
        return err(KR_E_FORMAT, "'%s': header of %llu bytes runs past the end of the %zu-byte file", path.c_str(),
                   (unsigned long long)hlen, s.size);
    s.data_off = 8 + hlen;
    JVal root;
    std::string why;
    if (!JParser((const char *)b + 8, (size_t)hlen).parse(root, why))
        return err(KR_E_FORMAT, "'%s': header JSON: %s", path.c_str(), why.c_str());
    if (root.kind != JVal::Obj) return err(KR_E_FORMAT, "'%s': header is not a JSON object", path.c_str());
    const uint64_t data_bytes = s.size - s.data_off;
    for (const auto &kv : root.obj) {
        const std::string &name = kv.first;
        if (name == "__metadata__") continue;
        const JVal &e = kv.second;
        const JVal *dt = e.kind == JVal::Obj ? e.get("dtype") : nullptr;
        const JVal *sh = e.kind == JVal::Obj ? e.get("shape") : nullptr;
        const JVal *of = e.kind == JVal::Obj ? e.get("data_offsets") : nullptr;
        if (!dt || dt->kind != JVal::Str || !sh || sh->kind != JVal::Arr || !of || of->kind != JVal::Arr ||
            of->arr.size() != 2 || !of->arr[0].is_uint || !of->arr[1].is_uint)
            return err(KR_E_FORMAT, "'%s': entry '%s' needs dtype, shape and data_offsets [begin, end]", path.c_str(),
                       name.c_str());
        const DTypeInfo *d = dtype_by_name(dt->s);
        if (!d) return err(KR_E_FORMAT, "'%s': unsupported safetensors dtype '%s' of '%s'", path.c_str(), dt->s.c_str(),
                           name.c_str());
        Tensor t;
        t.dtype = d->code;
        t.shard = shard_index;
        uint64_t elems = 1;
        if (sh->arr.size() > KR_MAX_DIMS)
            return err(KR_E_FORMAT, "'%s': '%s' has %zu dimensions (at most %d)", path.c_str(), name.c_str(),
                       sh->arr.size(), KR_MAX_DIMS);
        for (const JVal &x : sh->arr) {
            if (!x.is_uint) return err(KR_E_FORMAT, "'%s': '%s' has a non-integer dimension", path.c_str(), name.c_str());
            if (x.u != 0 && elems > UINT64_MAX / x.u)
                return err(KR_E_FORMAT, "'%s': '%s' has too many elements", path.c_str(), name.c_str());
            elems *= x.u;
            t.shape.push_back(x.u);
        }
        const uint64_t b0 = of->arr[0].u, b1 = of->arr[1].u;
        if (b1 < b0)
            return err(KR_E_FORMAT, "'%s': '%s' data_offsets end %llu < begin %llu", path.c_str(), name.c_str(),
                       (unsigned long long)b1, (unsigned long long)b0);
        t.off = b0;
        t.len = b1 - b0;
        // TensorDescriptor::validate: bytes == blocks(elements) * block bytes
        const uint64_t need = (elems + d->block_elems - 1) / d->block_elems * d->block_bytes;
        if (t.len != need)
            return err(KR_E_FORMAT, "'%s': '%s' holds %llu bytes, its dtype %s and shape need %llu", path.c_str(),
                       name.c_str(), (unsigned long long)t.len, d->name, (unsigned long long)need);
        if (b1 > data_bytes)
            return err(KR_E_FORMAT, "'%s': tensor '%s' exceeds the file (%llu > %llu data bytes)", path.c_str(),
                       name.c_str(), (unsigned long long)b1, (unsigned long long)data_bytes);
        h.tensors.emplace(name, std::move(t));
    }
    return KR_OK;
}

bool is_dir(const std::string &p) {
    struct stat st;
    return stat(p.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}
bool exists(const std::string &p) {
    struct stat st;
    return stat(p.c_str(), &st) == 0;
}

}  // namespace

struct kr_archive {
    std::vector<Shard> shards;
    std::map<std::string, Tensor> tensors;
    std::vector<std::string> names;  // sorted
    ~kr_archive() {
        for (auto &s : shards) unmap(s);
    }
    const Tensor *find(const std::string &n) const {
        auto it = tensors.find(n);
        return it == tensors.end() ? nullptr : &it->second;
    }
    const uint8_t *data(const Tensor &t) const {
        return (const uint8_t *)shards[t.shard].map + shards[t.shard].data_off + t.off;
    }
};

namespace {

// ShardedCheckpointLoader::open_sharded (safetensors_loader.rs:174-196): the weight map names
// every tensor and its shard; every named tensor must be in the header of its shard.
int open_sharded(const std::string &dir, const std::string &index_path, kr_archive &a) {
    Shard idx;
    if (int rc = map_file(index_path, idx)) return rc;
    JVal root;
    std::string why;
    const bool parsed = JParser((const char *)idx.map, idx.size).parse(root, why);
    unmap(idx);
    if (!parsed) return err(KR_E_FORMAT, "'%s': %s", index_path.c_str(), why.c_str());
    const JVal *wm = root.kind == JVal::Obj ? root.get("weight_map") : nullptr;
    if (!wm || wm->kind != JVal::Obj) return err(KR_E_FORMAT, "'%s': no weight_map object", index_path.c_str());
    std::map<std::string, int> shard_of_file;
    std::vector<Header> headers;
    for (const auto &kv : wm->obj) {
        if (kv.second.kind != JVal::Str) return err(KR_E_FORMAT, "'%s': weight_map values must be file names", index_path.c_str());
        const std::string &file = kv.second.s;
        if (file.empty() || file.find('/') != std::string::npos || file == "." || file == "..")
            return err(KR_E_FORMAT, "'%s': shard name '%s' is not a plain file name", index_path.c_str(), file.c_str());
        if (!shard_of_file.count(file)) {
            const int si = (int)a.shards.size();
            a.shards.emplace_back();
            a.shards.back().name = file;
            headers.emplace_back();
            if (int rc = parse_header(dir + "/" + file, a.shards.back(), si, headers.back())) return rc;
            shard_of_file[file] = si;
        }
    }
    for (const auto &kv : wm->obj) {
        const int si = shard_of_file[kv.second.s];
        auto it = headers[si].tensors.find(kv.first);
        if (it == headers[si].tensors.end())
            return err(KR_E_FORMAT, "index names '%s' in shard '%s', whose header does not hold it", kv.first.c_str(),
                       kv.second.s.c_str());
        a.tensors.emplace(kv.first, it->second);
    }
    return KR_OK;
}

int open_single(const std::string &file, const std::string &shard_name, kr_archive &a) {
    a.shards.emplace_back();
    a.shards.back().name = shard_name;
    Header h;
    if (int rc = parse_header(file, a.shards.back(), 0, h)) return rc;
    a.tensors = std::move(h.tensors);
    return KR_OK;
}

std::string base_name(const std::string &p) {
    const size_t i = p.find_last_of('/');
    return i == std::string::npos ? p : p.substr(i + 1);
}

// require_q4_weight (encoder.rs:332-418) and the dry run of pack_mlx_affine_q4_group64
// (safetensors_loader.rs:221-273).  On success: path 1 (one Q4_G64 tensor) or 2 (MLX triplet).
struct Q4Source {
    int path = 0;
    const Tensor *w = nullptr, *s = nullptr, *b = nullptr;
    std::string wname;
};

int find_q4(const kr_archive &a, const std::string &prefix, uint32_t n, uint32_t k, Q4Source &src) {
    if (n == 0 || k == 0 || k % 64 != 0)
        return err(KR_E_SHAPE, "'%s': shape [%u, %u] needs n > 0 and k a positive multiple of 64", prefix.c_str(), n, k);
    const uint64_t blocks = (uint64_t)n * (k / 64);
    const std::string sname = prefix + ".scales", bname = prefix + ".biases";
    const Tensor *s = a.find(sname), *b = a.find(bname);
    for (const std::string &wname : {prefix + ".weight", prefix}) {
        const Tensor *w = a.find(wname);
        if (!w) continue;
        if (w->dtype == KR_ST_Q4_G64) {  // Path A
            if (w->shape != std::vector<uint64_t>{n, k})
                return err(KR_E_FORMAT, "tensor '%s' of dtype Q4_G64 has a shape other than the expected [%u, %u]",
                           wname.c_str(), n, k);
            src = Q4Source{1, w, nullptr, nullptr, wname};
            return KR_OK;
        }
        if (!s || !b) continue;  // not a triplet under this name: try the bare prefix
        // Path B: the MLX triplet
        if (w->dtype != KR_ST_U32 && w->dtype != KR_ST_U8)
            return err(KR_E_FORMAT, "MLX weight tensor '%s' has dtype %s; expected packed U32 (or U8) nibbles",
                       wname.c_str(), dtype_by_code(w->dtype)->name);
        if (w->len != blocks * 32)
            return err(KR_E_FORMAT, "MLX weight tensor '%s' byte length %llu does not match expected %llu", wname.c_str(),
                       (unsigned long long)w->len, (unsigned long long)(blocks * 32));
        for (const auto &p : {std::make_pair(&sname, s), std::make_pair(&bname, b)}) {
            if (!is_float(p.second->dtype))
                return err(KR_E_FORMAT, "MLX tensor '%s' has dtype %s; expected float", p.first->c_str(),
                           dtype_by_code(p.second->dtype)->name);
            if (p.second->dtype == KR_ST_F32)
                return err(KR_E_FORMAT,
                           "MLX tensor '%s' is F32: the repack takes 2-byte BF16 or F16 scales and biases only",
                           p.first->c_str());
            if (p.second->len != blocks * 2)
                return err(KR_E_FORMAT, "MLX tensor '%s' holds %llu bytes; %llu groups need %llu", p.first->c_str(),
                           (unsigned long long)p.second->len, (unsigned long long)blocks,
                           (unsigned long long)(blocks * 2));
        }
        src = Q4Source{2, w, s, b, wname};
        return KR_OK;
    }
    return err(KR_E_MISSING,
               "checkpoint is missing expected weight '%s' (a Q4_G64 tensor, or an MLX .weight/.scales/.biases triplet)",
               prefix.c_str());
}

int find_float_vector(const kr_archive &a, const std::string &name, uint64_t len, const Tensor *&t) {
    t = a.find(name);
    if (!t) return err(KR_E_MISSING, "checkpoint is missing '%s'", name.c_str());
    if (!is_float(t->dtype))
        return err(KR_E_FORMAT, "tensor '%s' has dtype %s; expected floating point", name.c_str(),
                   dtype_by_code(t->dtype)->name);
    if (t->shape != std::vector<uint64_t>{len})
        return err(KR_E_FORMAT, "tensor '%s' does not have the expected shape [%llu]", name.c_str(),
                   (unsigned long long)len);
    return KR_OK;
}

int hip_rc(hipError_t e, const char *what) {
    return e == hipSuccess ? KR_OK : err(KR_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace

extern "C" {

int kr_archive_open(const char *path, kr_archive **out) {
    if (!path || !out) return err(KR_E_INVALID, "path/out must be non-NULL");
    *out = nullptr;
    std::unique_ptr<kr_archive> a(new kr_archive());
    const std::string p(path);
    int rc;
    if (is_dir(p)) {
        const std::string index = p + "/model.safetensors.index.json";
        rc = exists(index) ? open_sharded(p, index, *a) : open_single(p + "/model.safetensors", "model.safetensors", *a);
    } else {
        rc = open_single(p, base_name(p), *a);
    }
    if (rc) return rc;
    for (const auto &kv : a->tensors) a->names.push_back(kv.first);
    *out = a.release();
    return ok();
}

void kr_archive_close(kr_archive *a) { delete a; }

size_t kr_archive_tensor_count(const kr_archive *a) { return a ? a->names.size() : 0; }

const char *kr_archive_tensor_name(const kr_archive *a, size_t i) {
    return (a && i < a->names.size()) ? a->names[i].c_str() : nullptr;
}

int kr_archive_tensor(const kr_archive *a, const char *name, kr_tensor_info *info) {
    if (!a || !name || !info) return err(KR_E_INVALID, "archive/name/info must be non-NULL");
    const Tensor *t = a->find(name);
    if (!t) return err(KR_E_MISSING, "tensor '%s' is not in the archive", name);
    memset(info, 0, sizeof(*info));
    info->dtype = t->dtype;
    info->ndim = (uint32_t)t->shape.size();
    for (size_t i = 0; i < t->shape.size(); ++i) info->shape[i] = t->shape[i];
    info->byte_len = t->len;
    info->data = a->data(*t);
    info->shard = a->shards[t->shard].name.c_str();
    return ok();
}

int kr_archive_check_q4(const kr_archive *a, const char *prefix, uint32_t n, uint32_t k, int *path_out) {
    if (!a || !prefix) return err(KR_E_INVALID, "archive/prefix must be non-NULL");
    Q4Source src;
    if (int rc = find_q4(*a, prefix, n, k, src)) return rc;
    if (path_out) *path_out = src.path;
    return ok();
}

int kr_archive_q4_staging_bytes(const kr_archive *a, const char *prefix, uint32_t n, uint32_t k, size_t *bytes) {
    if (!a || !prefix || !bytes) return err(KR_E_INVALID, "archive/prefix/bytes must be non-NULL");
    Q4Source src;
    if (int rc = find_q4(*a, prefix, n, k, src)) return rc;
    *bytes = src.path == 1 ? (size_t)src.w->len : 0;
    return ok();
}

int kr_archive_load_q4(const kr_archive *a, const char *prefix, uint32_t n, uint32_t k, uint32_t *qw,
                       uint16_t *scales, uint16_t *biases, void *staging, size_t staging_bytes, void *stream) {
    if (!a || !prefix) return err(KR_E_INVALID, "archive/prefix must be non-NULL");
    if (!qw || !scales || !biases) return err(KR_E_INVALID, "qw/scales/biases must be non-NULL");
    if ((uintptr_t)qw % 16 || (uintptr_t)scales % 2 || (uintptr_t)biases % 2)
        return err(KR_E_ALIGN, "qw must be 16-byte aligned, scales/biases 2-byte aligned");
    Q4Source src;
    if (int rc = find_q4(*a, prefix, n, k, src)) return rc;
    hipStream_t s = (hipStream_t)stream;
    const size_t groups = (size_t)n * (k / 64);
    if (src.path == 1) {
        if (!staging || staging_bytes < src.w->len)
            return err(KR_E_WORKSPACE, "'%s': %llu bytes of device staging required, %zu given", src.wname.c_str(),
                       (unsigned long long)src.w->len, staging_bytes);
        if ((uintptr_t)staging % 4) return err(KR_E_ALIGN, "staging must be 4-byte aligned");
        if (int rc = hip_rc(hipMemcpyAsync(staging, a->data(*src.w), src.w->len, hipMemcpyHostToDevice, s),
                            "copying Q4_G64 blocks"))
            return rc;
        if (int rc = kr_q4_from_blocks36(staging, n, k, qw, scales, biases, stream)) return rc;
    } else {
        if (int rc = hip_rc(hipMemcpyAsync(qw, a->data(*src.w), src.w->len, hipMemcpyHostToDevice, s),
                            "copying MLX nibbles"))
            return rc;
        const std::pair<const Tensor *, uint16_t *> planes[2] = {{src.s, scales}, {src.b, biases}};
        for (const auto &pl : planes) {
            if (int rc = hip_rc(hipMemcpyAsync(pl.second, a->data(*pl.first), groups * 2, hipMemcpyHostToDevice, s),
                                "copying MLX scales/biases"))
                return rc;
            if (pl.first->dtype == KR_ST_F16)  // parse_half_endian(is_f16): bf16_rne(f16_to_f32), on the device
                if (int rc = kr_f16_to_bf16(pl.second, pl.second, groups, stream)) return rc;
        }
    }
    if (int rc = hip_rc(hipStreamSynchronize(s), "kr_archive_load_q4")) return rc;
    return ok();
}

int kr_archive_load_bf16(const kr_archive *a, const char *name, uint64_t len, uint16_t *out, void *stream) {
    if (!a || !name || !out) return err(KR_E_INVALID, "archive/name/out must be non-NULL");
    if ((uintptr_t)out % 2) return err(KR_E_ALIGN, "out must be 2-byte aligned");
    const Tensor *t = nullptr;
    if (int rc = find_float_vector(*a, name, len, t)) return rc;
    std::vector<uint16_t> host((size_t)len);
    const uint8_t *d = a->data(*t);
    for (size_t i = 0; i < (size_t)len; ++i) {
        if (t->dtype == KR_ST_BF16) {
            memcpy(&host[i], d + 2 * i, 2);
        } else if (t->dtype == KR_ST_F16) {
            uint16_t h;
            memcpy(&h, d + 2 * i, 2);
            host[i] = f32_to_bf16(f16_to_f32(h));
        } else {
            float f;
            memcpy(&f, d + 4 * i, 4);
            host[i] = f32_to_bf16(f);
        }
    }
    hipStream_t s = (hipStream_t)stream;
    if (int rc = hip_rc(hipMemcpyAsync(out, host.data(), (size_t)len * 2, hipMemcpyHostToDevice, s), name)) return rc;
    if (int rc = hip_rc(hipStreamSynchronize(s), "kr_archive_load_bf16")) return rc;
    return ok();
}

int kr_checkpoint_validate_dense(const kr_archive *a, const kr_dense_model_desc *d) {
    if (!a || !d) return err(KR_E_INVALID, "archive/desc must be non-NULL");
    if (!d->hidden || !d->intermediate || !d->layers || !d->vocab || !d->q_heads || !d->kv_heads || !d->head_dim ||
        d->q_heads % d->kv_heads)
        return err(KR_E_INVALID, "invalid architecture descriptor: sizes must be positive and q_heads a multiple of kv_heads");
    const uint32_t h = d->hidden, qd = d->q_heads * d->head_dim, kvd = d->kv_heads * d->head_dim;
    Q4Source src;
    const Tensor *t = nullptr;
    if (int rc = find_q4(*a, "model.embed_tokens", d->vocab, h, src)) return rc;
    if (int rc = find_float_vector(*a, "model.norm.weight", h, t)) return rc;
    if (!d->tie_word_embeddings)
        if (int rc = find_q4(*a, "lm_head", d->vocab, h, src)) return rc;
    for (uint32_t l = 0; l < d->layers; ++l) {
        const std::string p = "model.layers." + std::to_string(l);
        if (int rc = find_float_vector(*a, p + ".input_layernorm.weight", h, t)) return rc;
        if (int rc = find_float_vector(*a, p + ".post_attention_layernorm.weight", h, t)) return rc;
        const struct {
            const char *suffix;
            uint32_t n, k;
        } proj[] = {{".self_attn.q_proj", qd, h},          {".self_attn.k_proj", kvd, h},
                    {".self_attn.v_proj", kvd, h},         {".self_attn.o_proj", h, qd},
                    {".mlp.gate_proj", d->intermediate, h}, {".mlp.up_proj", d->intermediate, h},
                    {".mlp.down_proj", h, d->intermediate}};
        for (const auto &pr : proj)
            if (int rc = find_q4(*a, p + pr.suffix, pr.n, pr.k, src)) return rc;
        if (d->qkv_bias) {
            if (int rc = find_float_vector(*a, p + ".self_attn.q_proj.bias", qd, t)) return rc;
            if (int rc = find_float_vector(*a, p + ".self_attn.k_proj.bias", kvd, t)) return rc;
            if (int rc = find_float_vector(*a, p + ".self_attn.v_proj.bias", kvd, t)) return rc;
        }
    }
    return ok();
}

}  // extern "C"
