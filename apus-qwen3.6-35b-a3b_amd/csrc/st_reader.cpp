// st_reader.cpp -- the weight container reader: safetensors shards and the
// model.safetensors.index.json shard map, and loaders that put one GDN or
// one gated-GQA layer's hot-path weights on the device.
//
// The format (the reference's c/st.h:8-12): an 8-byte little-endian header
// length N, N bytes of JSON {"<name>": {"dtype", "shape", "data_offsets":
// [a, b]}, "__metadata__": {...}}, then the payloads, offsets relative to
// the end of the header. A directory holds model.safetensors.index.json
// {"weight_map": {"<name>": "<shard file>"}} and the shards (c/st.h:
// 77-89). Shards are opened header-only and a tensor is read with pread
// when asked for, into the caller's memory (nothing is cached: the layer
// loaders read each hot weight once on its way to the device).
//
// Names follow the reference loader (c/model.h:66-78, 440-490):
//   model.language_model.layers.{L}.linear_attn.conv1d.weight [C,1,4] BF16
//   ...linear_attn.norm.weight [dv] BF16, ...linear_attn.{A_log,dt_bias}
//   [hv] F32 (BF16 widened, c/model.h:249-275)
//   ...self_attn.{q,k}_norm.weight [d] BF16
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/apus_hip.h"
#include "apus_rt.h"

using namespace apus;

namespace {

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) ----
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    double num = 0;
    bool b = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json *get(const char *k) const {
        for (auto &p : obj)
            if (p.first == k) return &p.second;
        return nullptr;
    }
};

struct Parser {
    const char *p, *end;
    std::string err;
    int depth = 0;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool fail(const char *m) {
        if (err.empty()) err = m;
        return false;
    }
    bool lit(const char *s) {
        const size_t n = strlen(s);
        if ((size_t)(end - p) < n || memcmp(p, s, n) != 0) return fail("bad literal");
        p += n;
        return true;
    }
    static void utf8(std::string &o, uint32_t c) {
        if (c < 0x80) {
            o += (char)c;
        } else if (c < 0x800) {
            o += (char)(0xC0 | (c >> 6));
            o += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            o += (char)(0xE0 | (c >> 12));
            o += (char)(0x80 | ((c >> 6) & 0x3F));
            o += (char)(0x80 | (c & 0x3F));
        } else {
            o += (char)(0xF0 | (c >> 18));
            o += (char)(0x80 | ((c >> 12) & 0x3F));
            o += (char)(0x80 | ((c >> 6) & 0x3F));
            o += (char)(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t &v) {
        if (end - p < 4) return fail("short \\u escape");
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string &o) {
        if (p >= end || *p != '"') return fail("expected string");
        p++;
        while (p < end && *p != '"') {
            const char c = *p++;
            if ((unsigned char)c < 0x20) return fail("control character in string");
            if (c != '\\') {
                o += c;
                continue;
            }
            if (p >= end) return fail("unterminated escape");
            const char e = *p++;
            switch (e) {
            case '"': o += '"'; break;
            case '\\': o += '\\'; break;
            case '/': o += '/'; break;
            case 'b': o += '\b'; break;
            case 'f': o += '\f'; break;
            case 'n': o += '\n'; break;
            case 'r': o += '\r'; break;
            case 't': o += '\t'; break;
            case 'u': {
                uint32_t v;
                if (!hex4(v)) return false;
                if (v >= 0xD800 && v < 0xDC00) {          // surrogate pair
                    uint32_t lo;
                    if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return fail("lone surrogate");
                    p += 2;
                    if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate");
                    v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(o, v);
                break;
            }
            default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool number(double &v) {
        const char *s = p;
        if (p < end && (*p == '-' || *p == '+')) p++;
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' ||
                           *p == '-' || *p == '+'))
            p++;
        if (p == s) return fail("expected value");
        const std::string t(s, p);
        char *e = nullptr;
        v = strtod(t.c_str(), &e);
        if (!e || *e) return fail("bad number");
        return true;
    }
    bool value(Json &v) {
        if (++depth > 64) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end");
        bool ok = true;
        if (*p == '{') {
            v.kind = Json::Obj;
            p++;
            ws();
            if (p < end && *p == '}') {
                p++;
            } else {
                for (;;) {
                    ws();
                    std::pair<std::string, Json> kv;
                    if (!string(kv.first)) return false;
                    ws();
                    if (p >= end || *p != ':') return fail("expected ':'");
                    p++;
                    if (!value(kv.second)) return false;
                    v.obj.push_back(std::move(kv));
                    ws();
                    if (p < end && *p == ',') { p++; continue; }
                    if (p < end && *p == '}') { p++; break; }
                    return fail("expected ',' or '}'");
                }
            }
        } else if (*p == '[') {
            v.kind = Json::Arr;
            p++;
            ws();
            if (p < end && *p == ']') {
                p++;
            } else {
                for (;;) {
                    Json e;
                    if (!value(e)) return false;
                    v.arr.push_back(std::move(e));
                    ws();
                    if (p < end && *p == ',') { p++; continue; }
                    if (p < end && *p == ']') { p++; break; }
                    return fail("expected ',' or ']'");
                }
            }
        } else if (*p == '"') {
            v.kind = Json::Str;
            ok = string(v.str);
        } else if (*p == 't') {
            v.kind = Json::Bool;
            v.b = true;
            ok = lit("true");
        } else if (*p == 'f') {
            v.kind = Json::Bool;
            ok = lit("false");
        } else if (*p == 'n') {
            ok = lit("null");
        } else {
            v.kind = Json::Num;
            ok = number(v.num);
        }
        depth--;
        return ok;
    }
};

bool parse_json(const char *s, size_t n, Json &out, std::string &err) {
    Parser ps{s, s + n, {}, 0};
    if (!ps.value(out)) {
        err = ps.err;
        return false;
    }
    ps.ws();
    if (ps.p != ps.end) {
        err = "trailing bytes after JSON";
        return false;
    }
    return true;
}

// dtype names -> the codes of ApusHipStTensor.dtype (the reference's
// ApusStDtype order, c/st.h:44-48) and element sizes
struct DtypeInfo {
    const char *name;
    int code, size;
};
const DtypeInfo kDtypes[] = {{"I8", APUS_HIP_ST_I8, 1},        {"U8", APUS_HIP_ST_U8, 1},
                             {"F8_E8M0", APUS_HIP_ST_F8_E8M0, 1}, {"F8_E4M3", APUS_HIP_ST_F8_E4M3, 1},
                             {"BF16", APUS_HIP_ST_BF16, 2},    {"F16", APUS_HIP_ST_F16, 2},
                             {"F32", APUS_HIP_ST_F32, 4},      {"I32", APUS_HIP_ST_I32, 4},
                             {"I64", APUS_HIP_ST_I64, 8}};

struct Entry {
    ApusHipStTensor info;
    uint64_t off;     // absolute file offset of the payload
};

struct Shard {
    int fd = -1;
    std::string path;
    std::map<std::string, Entry> tensors;
    ~Shard() {
        if (fd >= 0) close(fd);
    }
};

bool read_at(int fd, void *dst, size_t n, uint64_t off) {
    char *d = (char *)dst;
    while (n) {
        const ssize_t r = pread(fd, d, n, (off_t)off);
        if (r <= 0) return false;
        d += r;
        n -= (size_t)r;
        off += (uint64_t)r;
    }
    return true;
}

int open_shard(const std::string &path, std::unique_ptr<Shard> &out) {
    auto sh = std::make_unique<Shard>();
    sh->path = path;
    sh->fd = open(path.c_str(), O_RDONLY);
    if (sh->fd < 0) return set_error(kErrArgument, "cannot open %s", path.c_str());
    struct stat st;
    if (fstat(sh->fd, &st) != 0) return set_error(kErrArgument, "cannot stat %s", path.c_str());
    const uint64_t fsz = (uint64_t)st.st_size;
    uint8_t h8[8];
    if (fsz < 8 || !read_at(sh->fd, h8, 8, 0))
        return set_error(kErrArgument, "%s is too small for a safetensors file", path.c_str());
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | h8[i];      // little-endian
    if (hlen > ((uint64_t)1 << 28) || 8 + hlen > fsz)
        return set_error(kErrArgument, "bad header length in %s", path.c_str());
    std::string hbuf(hlen, '\0');
    if (!read_at(sh->fd, &hbuf[0], hlen, 8))
        return set_error(kErrArgument, "cannot read the header of %s", path.c_str());
    Json hdr;
    std::string jerr;
    if (!parse_json(hbuf.data(), hbuf.size(), hdr, jerr) || hdr.kind != Json::Obj)
        return set_error(kErrArgument, "header JSON of %s: %s", path.c_str(),
                         jerr.empty() ? "not an object" : jerr.c_str());
    const uint64_t base = 8 + hlen;
    for (auto &kv : hdr.obj) {
        if (kv.first == "__metadata__") continue;
        const Json &m = kv.second;
        const Json *dt = m.get("dtype"), *shp = m.get("shape"), *offs = m.get("data_offsets");
        if (m.kind != Json::Obj || !dt || dt->kind != Json::Str || !shp ||
            shp->kind != Json::Arr || !offs || offs->kind != Json::Arr || offs->arr.size() != 2)
            return set_error(kErrArgument, "malformed entry %s in %s", kv.first.c_str(),
                             path.c_str());
        Entry e{};
        if (kv.first.size() >= sizeof e.info.name)
            return set_error(kErrArgument, "tensor name too long in %s", path.c_str());
        snprintf(e.info.name, sizeof e.info.name, "%s", kv.first.c_str());
        e.info.dtype = APUS_HIP_ST_OTHER;
        int esize = 0;
        for (auto &d : kDtypes)
            if (dt->str == d.name) {
                e.info.dtype = d.code;
                esize = d.size;
            }
        if (shp->arr.size() > APUS_HIP_ST_MAX_NDIM)
            return set_error(kErrArgument, "too many dimensions for %s", e.info.name);
        e.info.ndim = (int)shp->arr.size();
        // JSON numbers are doubles: a dimension or an offset is accepted
        // only as an integer below 2^53 (exact in a double, and the cast
        // below is then defined), and the element count must not overflow
        const double kMaxInt = 9007199254740992.0;   // 2^53
        auto is_index = [&](const Json &x) {
            return x.kind == Json::Num && x.num >= 0 && x.num < kMaxInt &&
                   x.num == (double)(uint64_t)x.num;
        };
        uint64_t nel = 1;
        for (int i = 0; i < e.info.ndim; i++) {
            const Json &x = shp->arr[i];
            if (!is_index(x)) return set_error(kErrArgument, "bad shape for %s", e.info.name);
            e.info.shape[i] = (int64_t)x.num;
            if (__builtin_mul_overflow(nel, (uint64_t)e.info.shape[i], &nel))
                return set_error(kErrArgument, "element count of %s overflows", e.info.name);
        }
        if (!is_index(offs->arr[0]) || !is_index(offs->arr[1]))
            return set_error(kErrArgument, "bad data_offsets for %s", e.info.name);
        const uint64_t a = (uint64_t)offs->arr[0].num, b = (uint64_t)offs->arr[1].num;
        if (b < a || base > fsz || b > fsz - base)
            return set_error(kErrArgument, "tensor %s lies past the end of %s", e.info.name,
                             path.c_str());
        e.info.nbytes = (size_t)(b - a);
        uint64_t want = 0;
        if (esize && (__builtin_mul_overflow(nel, (uint64_t)esize, &want) ||
                      (uint64_t)e.info.nbytes != want))
            return set_error(kErrArgument, "tensor %s: %zu bytes for %llu elements of %s",
                             e.info.name, e.info.nbytes, (unsigned long long)nel, dt->str.c_str());
        e.off = base + a;
        sh->tensors[kv.first] = e;
    }
    out = std::move(sh);
    return kOk;
}

}  // namespace

struct ApusHipSt {
    std::vector<std::unique_ptr<Shard>> shards;
    std::map<std::string, size_t> where;      // tensor name -> shard index
};

namespace {

int st_lookup(ApusHipSt *st, const char *name, const Entry **e, int *fd) {
    if (!st || !name) return set_error(kErrArgument, "NULL argument");
    auto it = st->where.find(name);
    if (it == st->where.end()) return set_error(kErrArgument, "tensor %s not in the container", name);
    Shard &sh = *st->shards[it->second];
    auto t = sh.tensors.find(name);
    if (t == sh.tensors.end())
        return set_error(kErrArgument, "tensor %s not in shard %s", name, sh.path.c_str());
    *e = &t->second;
    *fd = sh.fd;
    return kOk;
}

// Read a tensor of n elements as fp32 (F32 as is, BF16 widened exactly;
// the reference's A_log / dt_bias rule, c/model.h:249-275).
int st_read_f32(ApusHipSt *st, const std::string &name, size_t n, std::vector<float> &out) {
    const Entry *e;
    int fd;
    if (int r = st_lookup(st, name.c_str(), &e, &fd)) return r;
    out.assign(n, 0.0f);
    if (e->info.dtype == APUS_HIP_ST_F32 && e->info.nbytes == n * 4) {
        if (!read_at(fd, out.data(), n * 4, e->off)) return set_error(kErrArgument, "read failed");
        return kOk;
    }
    if (e->info.dtype == APUS_HIP_ST_BF16 && e->info.nbytes == n * 2) {
        std::vector<uint16_t> b(n);
        if (!read_at(fd, b.data(), n * 2, e->off)) return set_error(kErrArgument, "read failed");
        for (size_t i = 0; i < n; i++) {
            const uint32_t u = (uint32_t)b[i] << 16;
            memcpy(&out[i], &u, 4);
        }
        return kOk;
    }
    return set_error(kErrArgument, "%s: expected %zu F32 or BF16 elements", name.c_str(), n);
}

int st_read_bf16(ApusHipSt *st, const std::string &name, size_t n, std::vector<uint16_t> &out) {
    const Entry *e;
    int fd;
    if (int r = st_lookup(st, name.c_str(), &e, &fd)) return r;
    if (e->info.dtype != APUS_HIP_ST_BF16 || e->info.nbytes != n * 2)
        return set_error(kErrArgument, "%s: expected %zu BF16 elements", name.c_str(), n);
    out.resize(n);
    if (!read_at(fd, out.data(), n * 2, e->off)) return set_error(kErrArgument, "read failed");
    return kOk;
}

template <typename T> int to_device(const std::vector<T> &h, T **d) {
    APUS_HIP_TRY(hipMalloc((void **)d, h.size() * sizeof(T)));
    APUS_HIP_TRY(hipMemcpy(*d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return kOk;
}

std::string layer_name(int layer, const char *suffix) {
    char b[256];
    snprintf(b, sizeof b, "model.language_model.layers.%d.%s", layer, suffix);
    return b;
}

}  // namespace

extern "C" {

int apus_hip_st_open(const char *path, ApusHipSt **out) {
    if (!path || !out) return set_error(kErrArgument, "NULL argument");
    *out = nullptr;
    struct stat st;
    if (stat(path, &st) != 0) return set_error(kErrArgument, "cannot stat %s", path);
    auto set = std::make_unique<ApusHipSt>();
    if (!S_ISDIR(st.st_mode)) {
        std::unique_ptr<Shard> sh;
        if (int r = open_shard(path, sh)) return r;
        for (auto &kv : sh->tensors) set->where[kv.first] = 0;
        set->shards.push_back(std::move(sh));
        *out = set.release();
        return kOk;
    }
    // a directory: model.safetensors.index.json maps names to shard files
    const std::string dir = path, ipath = dir + "/model.safetensors.index.json";
    const int fd = open(ipath.c_str(), O_RDONLY);
    if (fd < 0) return set_error(kErrArgument, "cannot open %s", ipath.c_str());
    struct stat ist;
    if (fstat(fd, &ist) != 0 || ist.st_size > (1 << 28)) {
        close(fd);
        return set_error(kErrArgument, "bad index file %s", ipath.c_str());
    }
    std::string buf((size_t)ist.st_size, '\0');
    const bool ok = read_at(fd, &buf[0], buf.size(), 0);
    close(fd);
    Json idx;
    std::string jerr;
    if (!ok || !parse_json(buf.data(), buf.size(), idx, jerr) || idx.kind != Json::Obj)
        return set_error(kErrArgument, "index JSON %s: %s", ipath.c_str(),
                         jerr.empty() ? "not an object" : jerr.c_str());
    const Json *wm = idx.get("weight_map");
    if (!wm || wm->kind != Json::Obj) return set_error(kErrArgument, "no weight_map in %s", ipath.c_str());
    std::map<std::string, size_t> shard_of_file;
    for (auto &kv : wm->obj) {
        if (kv.second.kind != Json::Str || kv.second.str.find('/') != std::string::npos)
            return set_error(kErrArgument, "bad shard name for %s", kv.first.c_str());
        auto it = shard_of_file.find(kv.second.str);
        if (it == shard_of_file.end()) {
            std::unique_ptr<Shard> sh;
            if (int r = open_shard(dir + "/" + kv.second.str, sh)) return r;
            it = shard_of_file.emplace(kv.second.str, set->shards.size()).first;
            set->shards.push_back(std::move(sh));
        }
        if (!set->shards[it->second]->tensors.count(kv.first))
            return set_error(kErrArgument, "index names %s in %s, which does not hold it",
                             kv.first.c_str(), kv.second.str.c_str());
        set->where[kv.first] = it->second;
    }
    *out = set.release();
    return kOk;
}

int apus_hip_st_close(ApusHipSt *st) {
    delete st;
    return kOk;
}

size_t apus_hip_st_ntensors(const ApusHipSt *st) { return st ? st->where.size() : 0; }

int apus_hip_st_find(ApusHipSt *st, const char *name, ApusHipStTensor *info) {
    const Entry *e;
    int fd;
    if (int r = st_lookup(st, name, &e, &fd)) return r;
    if (info) *info = e->info;
    return kOk;
}

int apus_hip_st_read(ApusHipSt *st, const char *name, void *dst, size_t cap) {
    const Entry *e;
    int fd;
    if (int r = st_lookup(st, name, &e, &fd)) return r;
    if (!dst || cap < e->info.nbytes)
        return set_error(kErrArgument, "%s needs %zu bytes", name, e->info.nbytes);
    if (!read_at(fd, dst, e->info.nbytes, e->off))
        return set_error(kErrArgument, "read of %s failed", name);
    return kOk;
}

int apus_hip_gdn_layer_load(ApusHipSt *st, int layer, size_t hk, size_t hv, size_t dk, size_t dv,
                            ApusHipGdnLayer *out) {
    APUS_READY();
    if (!out || layer < 0) return set_error(kErrArgument, "bad argument");
    const size_t cd = 2 * hk * dk + hv * dv;
    std::vector<uint16_t> conv, onorm;
    std::vector<float> alog, dtb;
    if (int r = st_read_bf16(st, layer_name(layer, "linear_attn.conv1d.weight"), cd * 4, conv)) return r;
    if (int r = st_read_bf16(st, layer_name(layer, "linear_attn.norm.weight"), dv, onorm)) return r;
    if (int r = st_read_f32(st, layer_name(layer, "linear_attn.A_log"), hv, alog)) return r;
    if (int r = st_read_f32(st, layer_name(layer, "linear_attn.dt_bias"), hv, dtb)) return r;
    uint16_t *dc = nullptr, *dn = nullptr;
    float *da = nullptr, *dd = nullptr;
    int r = to_device(conv, &dc);
    if (!r) r = to_device(onorm, &dn);
    if (!r) r = to_device(alog, &da);
    if (!r) r = to_device(dtb, &dd);
    if (r) {
        (void)hipFree(dc); (void)hipFree(dn); (void)hipFree(da); (void)hipFree(dd);
        return r;
    }
    *out = ApusHipGdnLayer{hk, hv, dk, dv, dc, da, dd, dn};
    return kOk;
}

int apus_hip_attn_layer_load(ApusHipSt *st, int layer, size_t nh, size_t nkv, size_t d,
                             size_t rot, double theta, ApusHipAttnLayer *out) {
    APUS_READY();
    if (!out || layer < 0) return set_error(kErrArgument, "bad argument");
    std::vector<uint16_t> qn, kn;
    if (int r = st_read_bf16(st, layer_name(layer, "self_attn.q_norm.weight"), d, qn)) return r;
    if (int r = st_read_bf16(st, layer_name(layer, "self_attn.k_norm.weight"), d, kn)) return r;
    uint16_t *dq = nullptr, *dk = nullptr;
    int r = to_device(qn, &dq);
    if (!r) r = to_device(kn, &dk);
    if (r) {
        (void)hipFree(dq); (void)hipFree(dk);
        return r;
    }
    *out = ApusHipAttnLayer{nh, nkv, d, rot, theta, dq, dk};
    return kOk;
}

int apus_hip_gdn_layer_free(ApusHipGdnLayer *L) {
    APUS_READY();
    if (!L) return kOk;
    (void)hipFree((void *)L->conv_w);
    (void)hipFree((void *)L->A_log);
    (void)hipFree((void *)L->dt_bias);
    (void)hipFree((void *)L->onorm_w);
    L->conv_w = L->onorm_w = nullptr;
    L->A_log = L->dt_bias = nullptr;
    return kOk;
}

int apus_hip_attn_layer_free(ApusHipAttnLayer *L) {
    APUS_READY();
    if (!L) return kOk;
    (void)hipFree((void *)L->qn_w);
    (void)hipFree((void *)L->kn_w);
    L->qn_w = L->kn_w = nullptr;
    return kOk;
}

}  // extern "C"
