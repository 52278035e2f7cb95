// GGUF v3 reader of the C ABI (Gguf::open / parse, src/gguf.rs:50-210, with
// the Tencent legacy-profile rules of :111-153) and the dense model loader
// (Model::from_gguf, src/model.rs:136-262, dense arm).
//
// The file is mapped read-only (or a caller's buffer is borrowed); every
// count, string, array and tensor extent is bounds-checked before use, in
// the reference's order and with its limits: a count may not exceed what the
// remaining bytes could hold at its element's minimum size, strings are at
// most 64 MiB of valid UTF-8, arrays at most 16,000,000 elements of a scalar
// or string type, float metadata is finite, booleans are 0 or 1, metadata
// keys and tensor names are unique, tensor offsets are aligned, extents lie
// in the file and do not overlap, and a row holds whole blocks. Type ids 40
// and 42 are Q2_0C / STQ1_0 only under their Tencent profiles; under the
// automatic profile a file carrying them is accepted only if its SHA-256 is
// one of the two known exports.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "hyq_abi.hpp"

using namespace hyq;

namespace {

// ---- SHA-256 (FIPS 180-4) ----
struct Sha256 {
    uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                     0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    uint8_t buf[64];
    size_t fill = 0;
    uint64_t total = 0;

    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

    void block(const uint8_t *p)
    {
        static const uint32_t K[64] = {
            0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u,
            0x923f82a4u, 0xab1c5ed5u, 0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u,
            0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u, 0xe49b69c1u, 0xefbe4786u,
            0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
            0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u,
            0x06ca6351u, 0x14292967u, 0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u,
            0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u, 0xa2bfe8a1u, 0xa81a664bu,
            0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
            0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au,
            0x5b9cca4fu, 0x682e6ff3u, 0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u,
            0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 |
                   (uint32_t)p[4 * i + 2] << 8 | (uint32_t)p[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
            const uint32_t ch = (e & f) ^ (~e & g);
            const uint32_t t1 = k + S1 + ch + K[i] + w[i];
            const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
            const uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
            const uint32_t t2 = S0 + mj;
            k = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = b;
            b = a;
            a = t1 + t2;
        }
        h[0] += a;
        h[1] += b;
        h[2] += c;
        h[3] += d;
        h[4] += e;
        h[5] += f;
        h[6] += g;
        h[7] += k;
    }
    void update(const uint8_t *p, size_t n)
    {
        total += n;
        if (fill) {
            const size_t m = std::min(n, 64 - fill);
            memcpy(buf + fill, p, m);
            fill += m;
            p += m;
            n -= m;
            if (fill == 64) {
                block(buf);
                fill = 0;
            }
        }
        for (; n >= 64; p += 64, n -= 64) block(p);
        memcpy(buf, p, n);
        fill += n;
    }
    void finish(uint8_t out[32])
    {
        const uint64_t bits = total * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(len, 8);
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(h[i] >> (24 - 8 * j));
    }
};

std::string hex(const uint8_t *d, size_t n)
{
    static const char *x = "0123456789abcdef";
    std::string s;
    for (size_t i = 0; i < n; ++i) {
        s += x[d[i] >> 4];
        s += x[d[i] & 15];
    }
    return s;
}

// SHA-256 digests of the two known Tencent legacy exports (src/gguf.rs:14-15)
const char *STQ_SHA256 = "cc497fe8f033b52b3b8b00a7669e9661435432f9d4cd43f7ed24400c01507a93";
const char *Q2C_SHA256 = "dcc33bbae9b28d923c8c76a64f6157840841d26f8774f3dfd770d5fabeeb1cd7";

// Strict UTF-8 (no overlong forms, surrogates or code points past U+10FFFF).
bool valid_utf8(const uint8_t *s, size_t n)
{
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int len;
        uint32_t cp, min;
        if ((c & 0xE0) == 0xC0) len = 2, cp = c & 0x1F, min = 0x80;
        else if ((c & 0xF0) == 0xE0) len = 3, cp = c & 0x0F, min = 0x800;
        else if ((c & 0xF8) == 0xF0) len = 4, cp = c & 0x07, min = 0x10000;
        else return false;
        if (n - i < (size_t)len) return false;
        for (int k = 1; k < len; ++k) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = cp << 6 | (s[i + k] & 0x3F);
        }
        if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += len;
    }
    return true;
}

// One metadata value, with the accessors of serde_json::Value that the
// reference uses: as_u64 (non-negative integers), as_f64 (any number),
// as_bool, as_str; arrays keep their element type and length.
struct Meta {
    uint32_t kind = 0;
    bool is_uint = false, is_num = false, is_bool = false, is_str = false, is_array = false;
    uint64_t u = 0;
    double f = 0.0;
    bool b = false;
    std::string s;
    uint32_t elem = 0;
    uint64_t count = 0;
};

struct Reader {
    const uint8_t *p;
    size_t len, pos = 0;

    int take(size_t n, const uint8_t **out)
    {
        if (n > len - pos) return fail(HYQ_EINVAL, "truncated GGUF header");
        *out = p + pos;
        pos += n;
        return HYQ_OK;
    }
    int u32(uint32_t *v)
    {
        const uint8_t *b;
        int rc = take(4, &b);
        if (!rc) memcpy(v, b, 4);
        return rc;
    }
    int u64(uint64_t *v)
    {
        const uint8_t *b;
        int rc = take(8, &b);
        if (!rc) memcpy(v, b, 8);
        return rc;
    }
    // a count no larger than the remaining bytes can hold at `minimum` each
    int count(size_t minimum, uint64_t *n)
    {
        int rc = u64(n);
        if (rc) return rc;
        if (*n > (len - pos) / minimum) return fail(HYQ_EINVAL, "GGUF count exceeds file bounds");
        return HYQ_OK;
    }
    int string(std::string *s)
    {
        uint64_t n;
        int rc = count(1, &n);
        if (rc) return rc;
        if (n > 64ull * 1024 * 1024) return fail(HYQ_EINVAL, "GGUF string exceeds 64 MiB limit");
        const uint8_t *b;
        if ((rc = take((size_t)n, &b))) return rc;
        if (!valid_utf8(b, (size_t)n)) return fail(HYQ_EINVAL, "invalid GGUF UTF-8");
        s->assign((const char *)b, (size_t)n);
        return HYQ_OK;
    }
    // src/gguf.rs:337-388
    int value(uint32_t kind, Meta *m, bool in_array)
    {
        m->kind = kind;
        const uint8_t *b;
        int rc;
        auto sint = [&](int64_t v) {
            m->is_num = true;
            m->f = (double)v;
            if (v >= 0) {
                m->is_uint = true;
                m->u = (uint64_t)v;
            }
        };
        auto uint = [&](uint64_t v) {
            m->is_num = m->is_uint = true;
            m->u = v;
            m->f = (double)v;
        };
        switch (kind) {
        case 0:
            if ((rc = take(1, &b))) return rc;
            uint(b[0]);
            return HYQ_OK;
        case 1:
            if ((rc = take(1, &b))) return rc;
            sint((int8_t)b[0]);
            return HYQ_OK;
        case 2:
        case 3: {
            if ((rc = take(2, &b))) return rc;
            uint16_t v;
            memcpy(&v, b, 2);
            if (kind == 2) uint(v);
            else sint((int16_t)v);
            return HYQ_OK;
        }
        case 4:
        case 5: {
            uint32_t v;
            if ((rc = u32(&v))) return rc;
            if (kind == 4) uint(v);
            else sint((int32_t)v);
            return HYQ_OK;
        }
        case 6: {
            uint32_t v;
            if ((rc = u32(&v))) return rc;
            float x;
            memcpy(&x, &v, 4);
            if (!std::isfinite(x)) return fail(HYQ_EINVAL, "non-finite GGUF metadata");
            m->is_num = true;
            m->f = x;
            return HYQ_OK;
        }
        case 7:
            if ((rc = take(1, &b))) return rc;
            if (b[0] > 1) return fail(HYQ_EINVAL, "invalid GGUF boolean");
            m->is_bool = true;
            m->b = b[0] == 1;
            return HYQ_OK;
        case 8:
            m->is_str = true;
            return string(&m->s);
        case 9: {
            if (in_array) break; // element type 9 has no minimum size: unsupported
            uint32_t et;
            if ((rc = u32(&et))) return rc;
            size_t minimum;
            switch (et) {
            case 0: case 1: case 7: minimum = 1; break;
            case 2: case 3: minimum = 2; break;
            case 4: case 5: case 6: minimum = 4; break;
            case 8: case 10: case 11: case 12: minimum = 8; break;
            default: return fail(HYQ_EINVAL, "unsupported GGUF array element type %u", et);
            }
            uint64_t n;
            if ((rc = count(minimum, &n))) return rc;
            if (n > 16000000) return fail(HYQ_EINVAL, "GGUF array is too large");
            for (uint64_t i = 0; i < n; ++i) {
                Meta item;
                if ((rc = value(et, &item, true))) return rc;
            }
            m->is_array = true;
            m->elem = et;
            m->count = n;
            return HYQ_OK;
        }
        case 10:
        case 11: {
            uint64_t v;
            if ((rc = u64(&v))) return rc;
            if (kind == 10) uint(v);
            else sint((int64_t)v);
            return HYQ_OK;
        }
        case 12: {
            uint64_t v;
            if ((rc = u64(&v))) return rc;
            double x;
            memcpy(&x, &v, 8);
            if (!std::isfinite(x)) return fail(HYQ_EINVAL, "non-finite GGUF metadata");
            m->is_num = true;
            m->f = x;
            return HYQ_OK;
        }
        default:
            break;
        }
        return fail(HYQ_EINVAL, "unsupported GGUF metadata type %u", kind);
    }
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type_id = 0;
    int dtype = 0;
    size_t offset = 0, byte_len = 0;
};

const char *profile_name(int p)
{
    switch (p) {
    case HYQ_PROFILE_AUTO: return "Auto";
    case HYQ_PROFILE_STANDARD: return "Standard";
    case HYQ_PROFILE_TENCENT_Q2_0C: return "TencentQ2_0c";
    case HYQ_PROFILE_TENCENT_STQ1: return "TencentStq1";
    default: return "?";
    }
}

// DType::from_id (src/quant.rs:30-41); -1 if the id has no format under the profile
int dtype_from_id(uint32_t id, int profile)
{
    switch (id) {
    case 0: return HYQ_F32;
    case 1: return HYQ_F16;
    case 8: return HYQ_Q8_0;
    case 12: return HYQ_Q4_K;
    case 14: return HYQ_Q6_K;
    case 40: return profile == HYQ_PROFILE_TENCENT_Q2_0C ? HYQ_Q2_0C : -1;
    case 42: return profile == HYQ_PROFILE_TENCENT_STQ1 ? HYQ_STQ1_0 : -1;
    default: return -1;
    }
}

} // namespace

struct hyq_gguf {
    const uint8_t *data = nullptr;
    size_t len = 0;
    void *map = nullptr; // set when the file is mapped here
    int profile = HYQ_PROFILE_STANDARD;
    std::map<std::string, Meta> meta;
    std::vector<Tensor> tensors; // sorted by name
    ~hyq_gguf()
    {
        if (map) munmap(map, len);
    }
    const Tensor *find(const char *name) const
    {
        auto it = std::lower_bound(tensors.begin(), tensors.end(), name,
                                   [](const Tensor &t, const char *n) { return t.name < n; });
        return it != tensors.end() && it->name == name ? &*it : nullptr;
    }
    const Meta *get(const std::string &key) const
    {
        auto it = meta.find(key);
        return it == meta.end() ? nullptr : &it->second;
    }
};

namespace {

// Gguf::parse (src/gguf.rs:60-210)
int parse(hyq_gguf *g, int requested)
{
    Reader r{g->data, g->len};
    const uint8_t *magic;
    int rc = r.take(4, &magic);
    if (rc) return rc;
    if (memcmp(magic, "GGUF", 4)) return fail(HYQ_EINVAL, "not a GGUF file");
    uint32_t version;
    if ((rc = r.u32(&version))) return rc;
    if (version != 3) return fail(HYQ_EINVAL, "only GGUF v3 is supported");
    uint64_t tensor_count, kv_count;
    if ((rc = r.count(24, &tensor_count))) return rc;
    if ((rc = r.count(13, &kv_count))) return rc;
    for (uint64_t i = 0; i < kv_count; ++i) {
        std::string key;
        uint32_t kind;
        Meta m;
        if ((rc = r.string(&key)) || (rc = r.u32(&kind)) || (rc = r.value(kind, &m, false)))
            return rc;
        if (!g->meta.emplace(key, std::move(m)).second)
            return fail(HYQ_EINVAL, "duplicate metadata key %s", key.c_str());
    }
    uint64_t alignment = 32;
    if (const Meta *a = g->get("general.alignment")) {
        if (!a->is_uint) return fail(HYQ_EINVAL, "invalid GGUF alignment");
        alignment = a->u;
    }
    if (alignment == 0 || (alignment & (alignment - 1)) || alignment > 65536)
        return fail(HYQ_EINVAL, "invalid GGUF alignment %llu", (unsigned long long)alignment);
    if (const Meta *s = g->get("split.count"))
        if (!(s->is_uint && s->u == 1))
            return fail(HYQ_EINVAL, "split GGUF files are not supported; supply a merged file");

    std::vector<Tensor> raw;
    raw.reserve((size_t)tensor_count);
    for (uint64_t i = 0; i < tensor_count; ++i) {
        Tensor t;
        uint32_t rank;
        if ((rc = r.string(&t.name)) || (rc = r.u32(&rank))) return rc;
        if (rank < 1 || rank > 4)
            return fail(HYQ_EINVAL, "invalid rank for tensor %s", t.name.c_str());
        for (uint32_t k = 0; k < rank; ++k) {
            uint64_t d;
            if ((rc = r.u64(&d))) return rc;
            if (d == 0) return fail(HYQ_EINVAL, "zero dimension in tensor %s", t.name.c_str());
            t.dims.push_back(d);
        }
        uint64_t off;
        if ((rc = r.u32(&t.type_id)) || (rc = r.u64(&off))) return rc;
        if (off % alignment) return fail(HYQ_EINVAL, "unaligned tensor %s", t.name.c_str());
        t.offset = (size_t)off;
        raw.push_back(std::move(t));
    }
    if (r.pos > SIZE_MAX - (alignment - 1)) return fail(HYQ_EINVAL, "offset overflow");
    const size_t data_start = (r.pos + (alignment - 1)) & ~(size_t)(alignment - 1);
    if (data_start > g->len) return fail(HYQ_EINVAL, "missing tensor data");

    // the profile (src/gguf.rs:111-128)
    const bool legacy = std::any_of(raw.begin(), raw.end(), [](const Tensor &t) {
        return t.type_id == 40 || t.type_id == 42;
    });
    int profile = requested;
    if (requested == HYQ_PROFILE_AUTO && legacy) {
        uint8_t d[32];
        Sha256 h;
        h.update(g->data, g->len);
        h.finish(d);
        const std::string digest = hex(d, 32);
        if (digest == Q2C_SHA256) profile = HYQ_PROFILE_TENCENT_Q2_0C;
        else if (digest == STQ_SHA256) profile = HYQ_PROFILE_TENCENT_STQ1;
        else
            return fail(HYQ_EINVAL,
                        "ambiguous GGUF type 40/42 in an unrecognized file (SHA256 %s); use the "
                        "tencent-q2-0c or tencent-stq1 profile only for a known Tencent legacy "
                        "export",
                        digest.c_str());
    } else if (requested == HYQ_PROFILE_AUTO) {
        profile = HYQ_PROFILE_STANDARD;
    }
    // the Tencent rules (src/gguf.rs:129-153)
    if (profile == HYQ_PROFILE_TENCENT_Q2_0C || profile == HYQ_PROFILE_TENCENT_STQ1) {
        const Meta *arch = g->get("general.architecture");
        if (!(arch && arch->is_str && arch->s == "hunyuan-dense"))
            return fail(HYQ_EINVAL, "Tencent low-bit profiles require hunyuan-dense");
        const uint32_t id = profile == HYQ_PROFILE_TENCENT_Q2_0C ? 40 : 42;
        const uint64_t file_type = profile == HYQ_PROFILE_TENCENT_Q2_0C ? 39 : 41;
        const Meta *ft = g->get("general.file_type");
        if (!(ft && ft->is_uint && ft->u == file_type))
            return fail(HYQ_EINVAL, "incompatible Tencent general.file_type");
        if (!std::any_of(raw.begin(), raw.end(), [&](const Tensor &t) { return t.type_id == id; }))
            return fail(HYQ_EINVAL, "file has no tensors for selected Tencent profile");
        for (const Tensor &t : raw)
            if (t.type_id != 0 && t.type_id != 14 && t.type_id != id)
                return fail(HYQ_EINVAL, "unexpected mixed types in Tencent legacy export");
    }

    // types, sizes and extents (src/gguf.rs:154-201)
    std::vector<std::pair<std::pair<size_t, size_t>, std::string>> extents;
    for (Tensor &t : raw) {
        t.dtype = dtype_from_id(t.type_id, profile);
        if (t.dtype < 0)
            return fail(HYQ_EDTYPE, "tensor %s: unsupported GGUF tensor type %u for profile %s",
                        t.name.c_str(), t.type_id, profile_name(profile));
        const uint64_t bl = (uint64_t)block_len(t.dtype), bb = (uint64_t)block_bytes(t.dtype);
        if (t.dims[0] % bl)
            return fail(HYQ_EINVAL, "tensor %s has a partial quantization block in its row",
                        t.name.c_str());
        uint64_t elements = 1;
        for (uint64_t d : t.dims) {
            if (elements > UINT64_MAX / d) return fail(HYQ_EINVAL, "tensor element count overflow");
            elements *= d;
        }
        if (elements / bl > UINT64_MAX / bb) return fail(HYQ_EINVAL, "tensor byte count overflow");
        const uint64_t byte_len = elements / bl * bb;
        if (t.offset > SIZE_MAX - data_start) return fail(HYQ_EINVAL, "tensor offset overflow");
        const size_t offset = data_start + t.offset;
        if (byte_len > SIZE_MAX - offset) return fail(HYQ_EINVAL, "tensor end overflow");
        const size_t end = offset + (size_t)byte_len;
        if (end > g->len)
            return fail(HYQ_EINVAL, "truncated tensor %s: end %zu, file length %zu",
                        t.name.c_str(), end, g->len);
        t.offset = offset;
        t.byte_len = (size_t)byte_len;
        extents.push_back({{offset, end}, t.name});
    }
    std::sort(raw.begin(), raw.end(),
              [](const Tensor &a, const Tensor &b) { return a.name < b.name; });
    for (size_t i = 1; i < raw.size(); ++i)
        if (raw[i].name == raw[i - 1].name)
            return fail(HYQ_EINVAL, "duplicate tensor %s", raw[i].name.c_str());
    std::sort(extents.begin(), extents.end());
    for (size_t i = 1; i < extents.size(); ++i)
        if (extents[i - 1].first.second > extents[i].first.first)
            return fail(HYQ_EINVAL, "overlapping tensors %s and %s", extents[i - 1].second.c_str(),
                        extents[i].second.c_str());
    g->tensors = std::move(raw);
    g->profile = profile;
    return HYQ_OK;
}

int open_common(std::unique_ptr<hyq_gguf> g, int profile, hyq_gguf **out)
{
    if (profile < HYQ_PROFILE_AUTO || profile > HYQ_PROFILE_TENCENT_STQ1)
        return fail(HYQ_EINVAL, "unknown GGUF profile %d", profile);
    int rc = parse(g.get(), profile);
    if (rc) return rc;
    *out = g.release();
    return HYQ_OK;
}

void fill_info(const Tensor &t, hyq_gguf_tensor *o)
{
    memset(o, 0, sizeof *o);
    o->name = t.name.c_str();
    o->rank = (int)t.dims.size();
    for (size_t i = 0; i < t.dims.size(); ++i) o->dims[i] = t.dims[i];
    o->type_id = t.type_id;
    o->dtype = t.dtype;
    o->offset = t.offset;
    o->byte_len = t.byte_len;
}

} // namespace

extern "C" {

int hyq_sha256(const uint8_t *bytes, size_t len, uint8_t digest[32])
{
    if ((!bytes && len) || !digest) return fail(HYQ_EINVAL, "sha256: null argument");
    Sha256 h;
    if (len) h.update(bytes, len);
    h.finish(digest);
    return HYQ_OK;
}

int hyq_gguf_open(const char *path, int profile, hyq_gguf **out)
{
    if (!path || !out) return fail(HYQ_EINVAL, "gguf_open: null argument");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(HYQ_EINVAL, "opening %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return fail(HYQ_EINVAL, "opening %s: %s", path, strerror(errno));
    }
    auto g = std::make_unique<hyq_gguf>();
    g->len = (size_t)st.st_size;
    if (g->len) {
        void *m = mmap(nullptr, g->len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            close(fd);
            return fail(HYQ_EINVAL, "mapping %s: %s", path, strerror(errno));
        }
        g->map = m;
        g->data = (const uint8_t *)m;
    }
    close(fd);
    return open_common(std::move(g), profile, out);
}

int hyq_gguf_open_bytes(const uint8_t *bytes, size_t len, int profile, hyq_gguf **out)
{
    if ((!bytes && len) || !out) return fail(HYQ_EINVAL, "gguf_open_bytes: null argument");
    auto g = std::make_unique<hyq_gguf>();
    g->data = bytes;
    g->len = len;
    return open_common(std::move(g), profile, out);
}

void hyq_gguf_close(hyq_gguf *g) { delete g; }

int hyq_gguf_profile(const hyq_gguf *g) { return g ? g->profile : HYQ_EINVAL; }

size_t hyq_gguf_byte_len(const hyq_gguf *g) { return g ? g->len : 0; }

const uint8_t *hyq_gguf_bytes(const hyq_gguf *g) { return g ? g->data : nullptr; }

size_t hyq_gguf_tensor_count(const hyq_gguf *g) { return g ? g->tensors.size() : 0; }

int hyq_gguf_tensor_at(const hyq_gguf *g, size_t index, hyq_gguf_tensor *out)
{
    if (!g || !out) return fail(HYQ_EINVAL, "gguf_tensor_at: null argument");
    if (index >= g->tensors.size()) return fail(HYQ_EINVAL, "tensor index %zu", index);
    fill_info(g->tensors[index], out);
    return HYQ_OK;
}

int hyq_gguf_find_tensor(const hyq_gguf *g, const char *name, hyq_gguf_tensor *out)
{
    if (!g || !name || !out) return fail(HYQ_EINVAL, "gguf_tensor: null argument");
    const Tensor *t = g->find(name);
    if (!t) return fail(HYQ_EINVAL, "missing tensor %s", name);
    fill_info(*t, out);
    return HYQ_OK;
}

int hyq_gguf_meta_u64(const hyq_gguf *g, const char *key, uint64_t *out)
{
    if (!g || !key || !out) return fail(HYQ_EINVAL, "gguf_meta: null argument");
    const Meta *m = g->get(key);
    if (!m || !m->is_uint) return fail(HYQ_EINVAL, "missing or invalid integer metadata %s", key);
    *out = m->u;
    return HYQ_OK;
}

int hyq_gguf_meta_f64(const hyq_gguf *g, const char *key, double *out)
{
    if (!g || !key || !out) return fail(HYQ_EINVAL, "gguf_meta: null argument");
    const Meta *m = g->get(key);
    if (!m || !m->is_num) return fail(HYQ_EINVAL, "missing or invalid float metadata %s", key);
    *out = m->f;
    return HYQ_OK;
}

int hyq_gguf_meta_bool(const hyq_gguf *g, const char *key, int *out)
{
    if (!g || !key || !out) return fail(HYQ_EINVAL, "gguf_meta: null argument");
    const Meta *m = g->get(key);
    if (!m || !m->is_bool) return fail(HYQ_EINVAL, "missing or invalid boolean metadata %s", key);
    *out = m->b ? 1 : 0;
    return HYQ_OK;
}

int hyq_gguf_meta_str(const hyq_gguf *g, const char *key, const char **out, size_t *len)
{
    if (!g || !key || !out) return fail(HYQ_EINVAL, "gguf_meta: null argument");
    const Meta *m = g->get(key);
    if (!m || !m->is_str) return fail(HYQ_EINVAL, "missing or invalid string metadata %s", key);
    *out = m->s.c_str();
    if (len) *len = m->s.size();
    return HYQ_OK;
}

int hyq_gguf_meta_array(const hyq_gguf *g, const char *key, uint32_t *elem_type, uint64_t *count)
{
    if (!g || !key) return fail(HYQ_EINVAL, "gguf_meta: null argument");
    const Meta *m = g->get(key);
    if (!m || !m->is_array) return fail(HYQ_EINVAL, "missing or invalid array metadata %s", key);
    if (elem_type) *elem_type = m->elem;
    if (count) *count = m->count;
    return HYQ_OK;
}

int hyq_gguf_upload(hyq_ctx *ctx, const hyq_gguf *g, const char *name, hyq_weight **out)
{
    if (!ctx || !g || !name || !out) return fail(HYQ_EINVAL, "gguf_upload: null argument");
    const Tensor *t = g->find(name);
    if (!t) return fail(HYQ_EINVAL, "missing tensor %s", name);
    if (t->dims.size() != 2 && t->dims.size() != 3)
        return fail(HYQ_EINVAL, "%s: rank %zu is not a matrix or expert stack", name,
                    t->dims.size());
    return hyq_weight_upload(ctx, t->dtype, g->data + t->offset, t->byte_len, t->dims.data(),
                             (int)t->dims.size(), out);
}

int hyq_gguf_read_f32(hyq_ctx *ctx, const hyq_gguf *g, const char *name, float *out, size_t n)
{
    if (!ctx || !g || !name || !out) return fail(HYQ_EINVAL, "gguf_read_f32: null argument");
    const Tensor *t = g->find(name);
    if (!t) return fail(HYQ_EINVAL, "missing tensor %s", name);
    uint64_t elements = 1;
    for (uint64_t d : t->dims) elements *= d;
    if (elements != n)
        return fail(HYQ_EINVAL, "%s: %llu elements, buffer of %zu", name,
                    (unsigned long long)elements, n);
    return hyq_decode(ctx, t->dtype, g->data + t->offset, t->byte_len, out, n);
}

} // extern "C"

// ---------------------------------------------------------------------------
// Model::from_gguf (src/model.rs:136-262): the hunyuan-dense and hy_v3 arms
// ---------------------------------------------------------------------------
namespace {

struct Owned {
    std::vector<hyq_weight *> w;
    ~Owned()
    {
        for (hyq_weight *p : w) hyq_weight_release(p);
    }
};

// matrix(): the tensor with the expected GGUF shape (src/model.rs:769-773)
int matrix(hyq_ctx *ctx, const hyq_gguf *g, const std::string &name,
           std::initializer_list<uint64_t> shape, Owned &own, hyq_weight **out)
{
    const Tensor *t = g->find(name.c_str());
    if (!t) return fail(HYQ_EINVAL, "missing tensor %s", name.c_str());
    if (!std::equal(t->dims.begin(), t->dims.end(), shape.begin(), shape.end())) {
        std::string want, got;
        for (uint64_t d : shape) want += (want.empty() ? "" : ", ") + std::to_string(d);
        for (uint64_t d : t->dims) got += (got.empty() ? "" : ", ") + std::to_string(d);
        return fail(HYQ_EINVAL, "%s: expected GGUF shape [%s], got [%s]", name.c_str(),
                    want.c_str(), got.c_str());
    }
    int rc = hyq_gguf_upload(ctx, g, name.c_str(), out);
    if (!rc) own.w.push_back(*out);
    return rc;
}

// norm(): a finite vector of the expected length (src/model.rs:775-783)
int norm(hyq_ctx *ctx, const hyq_gguf *g, const std::string &name, size_t len,
         std::vector<float> &out)
{
    const Tensor *t = g->find(name.c_str());
    if (!t) return fail(HYQ_EINVAL, "missing tensor %s", name.c_str());
    if (t->dims.size() != 1 || t->dims[0] != len)
        return fail(HYQ_EINVAL, "%s: expected GGUF shape [%zu]", name.c_str(), len);
    out.resize(len);
    int rc = hyq_gguf_read_f32(ctx, g, name.c_str(), out.data(), len);
    if (rc) return rc;
    for (float v : out)
        if (!std::isfinite(v))
            return fail(HYQ_EINVAL, "non-finite normalization/router tensor %s", name.c_str());
    return HYQ_OK;
}

} // namespace

extern "C" int hyq_dense_from_gguf(hyq_ctx *ctx, const hyq_gguf *g, size_t context,
                                   hyq_dense **out)
{
    if (!ctx || !g || !out) return fail(HYQ_EINVAL, "dense_from_gguf: null argument");
    const Meta *arch = g->get("general.architecture");
    if (!arch || !arch->is_str)
        return fail(HYQ_EINVAL, "missing or invalid string metadata general.architecture");
    const std::string prefix = arch->s;
    const bool hyv3 = prefix == "hy_v3";
    if (prefix != "hunyuan-dense" && !hyv3)
        return fail(HYQ_EINVAL, "unsupported model architecture %s", prefix.c_str());
    auto integer = [&](const char *suffix, uint64_t *v) {
        return hyq_gguf_meta_u64(g, (prefix + "." + suffix).c_str(), v);
    };
    auto real = [&](const char *suffix, float *v) -> int {
        double d;
        int rc = hyq_gguf_meta_f64(g, (prefix + "." + suffix).c_str(), &d);
        if (rc) return rc;
        *v = (float)d;
        if (!std::isfinite(*v))
            return fail(HYQ_EINVAL, "non-finite metadata %s.%s", prefix.c_str(), suffix);
        return HYQ_OK;
    };
    uint64_t layers, hidden, heads, kv_heads, head_dim, ctx_len, value_len, ffn;
    float rope_base, eps;
    int rc;
    if ((rc = integer("block_count", &layers)) || (rc = integer("embedding_length", &hidden)) ||
        (rc = integer("attention.head_count", &heads)) ||
        (rc = integer("attention.head_count_kv", &kv_heads)) ||
        (rc = integer("attention.key_length", &head_dim)) ||
        (rc = integer("context_length", &ctx_len)) || (rc = real("rope.freq_base", &rope_base)) ||
        (rc = real("attention.layer_norm_rms_epsilon", &eps)))
        return rc;
    // vocab_size: the tokenizer's pieces (tokenizer.ggml.tokens, src/tokenizer.rs:54)
    uint64_t vocab;
    if ((rc = hyq_gguf_meta_array(g, "tokenizer.ggml.tokens", nullptr, &vocab))) return rc;
    if (!(layers > 0 && layers <= 1024 && hidden > 0))
        return fail(HYQ_EINVAL, "invalid model dimensions");
    if (!(heads > 0 && kv_heads > 0 && heads % kv_heads == 0))
        return fail(HYQ_EINVAL, "invalid grouped-query head counts");
    if (!(head_dim > 0 && head_dim % 2 == 0))
        return fail(HYQ_EINVAL, "invalid RoPE head dimension");
    if ((rc = integer("attention.value_length", &value_len))) return rc;
    if (value_len != head_dim)
        return fail(HYQ_EINVAL, "different key/value dimensions are not supported");
    if (!(ctx_len > 0 && rope_base > 0.f && eps > 0.f))
        return fail(HYQ_EINVAL, "invalid context, RoPE, or RMS settings");
    if (const Meta *sc = g->get(prefix + ".rope.scaling.type"))
        if (!(sc->is_str && sc->s == "none"))
            return fail(HYQ_EINVAL,
                        "GGUF must contain an effective RoPE base with no extra scaling");
    if (g->get(prefix + ".rope.dimension_count")) {
        uint64_t rd;
        if ((rc = integer("rope.dimension_count", &rd))) return rc;
        if (rd != head_dim) return fail(HYQ_EINVAL, "partial rotary embeddings are not supported");
    }
    if ((rc = integer("feed_forward_length", &ffn))) return rc;
    // Model::new_session: 0 < context <= context_length (src/model.rs:264-270)
    if (context == 0 || context > ctx_len)
        return fail(HYQ_EINVAL, "context must be between 1 and %llu", (unsigned long long)ctx_len);
    if (hidden > 0x7fffffff || ffn > 0x7fffffff || vocab > 0x7fffffff || heads > 4096)
        return fail(HYQ_EINVAL, "invalid model dimensions");

    hyq_dense_config cfg{};
    cfg.layers = (int)layers;
    cfg.hidden = (int)hidden;
    cfg.heads = (int)heads;
    cfg.kv_heads = (int)kv_heads;
    cfg.head_dim = (int)head_dim;
    cfg.ffn = (int)ffn;
    cfg.vocab = (int)vocab;
    cfg.rope_base = rope_base;
    cfg.rms_eps = eps;
    hyq_dense *m = nullptr;
    if ((rc = hyq_dense_create(ctx, &cfg, context, &m))) return rc;
    std::unique_ptr<hyq_dense, void (*)(hyq_dense *)> guard(m, hyq_dense_destroy);
    if (hyv3 && (rc = hyq_dense_set_architecture(m, HYQ_ARCH_HYV3))) return rc;
    Owned own;
    const uint64_t H = hidden, QL = heads * head_dim, KV = kv_heads * head_dim;
    hyq_weight *emb, *outw;
    if ((rc = matrix(ctx, g, "token_embd.weight", {H, vocab}, own, &emb))) return rc;
    if (g->find("output.weight")) {
        if ((rc = matrix(ctx, g, "output.weight", {H, vocab}, own, &outw))) return rc;
    } else {
        if (hyv3) return fail(HYQ_EINVAL, "HYV3 requires separate output weights");
        outw = emb; // tied (src/model.rs:194-202)
    }
    std::vector<float> onorm;
    if ((rc = norm(ctx, g, "output_norm.weight", H, onorm))) return rc;
    for (uint64_t i = 0; i < layers; ++i) {
        const std::string p = "blk." + std::to_string(i) + ".";
        hyq_weight *q, *k, *v, *o, *gate = nullptr, *up = nullptr, *down = nullptr;
        std::vector<float> an, fn, qn, kn;
        if ((rc = norm(ctx, g, p + "attn_norm.weight", H, an)) ||
            (rc = norm(ctx, g, p + "ffn_norm.weight", H, fn)) ||
            (rc = matrix(ctx, g, p + "attn_q.weight", {H, QL}, own, &q)) ||
            (rc = matrix(ctx, g, p + "attn_k.weight", {H, KV}, own, &k)) ||
            (rc = matrix(ctx, g, p + "attn_v.weight", {H, KV}, own, &v)) ||
            (rc = matrix(ctx, g, p + "attn_output.weight", {QL, H}, own, &o)) ||
            (rc = norm(ctx, g, p + "attn_q_norm.weight", head_dim, qn)) ||
            (rc = norm(ctx, g, p + "attn_k_norm.weight", head_dim, kn)))
            return rc;
        // HyV3: every layer after the first has an MoE FFN (src/model.rs:206-235)
        const bool moe = hyv3 && i > 0;
        if (!moe && ((rc = matrix(ctx, g, p + "ffn_gate.weight", {H, ffn}, own, &gate)) ||
                     (rc = matrix(ctx, g, p + "ffn_up.weight", {H, ffn}, own, &up)) ||
                     (rc = matrix(ctx, g, p + "ffn_down.weight", {ffn, H}, own, &down))))
            return rc;
        if ((rc = hyq_dense_set_layer(m, (int)i, q, k, v, o, gate, up, down, an.data(), fn.data(),
                                      qn.data(), kn.data())))
            return rc;
        if (!moe) continue;
        uint64_t experts, used, mid, shared, gating;
        float scale;
        int norm_w;
        if ((rc = integer("expert_count", &experts)) ||
            (rc = integer("expert_used_count", &used)) ||
            (rc = integer("expert_feed_forward_length", &mid)) ||
            (rc = integer("expert_shared_feed_forward_length", &shared)))
            return rc;
        if (!(experts > 0 && used > 0 && used <= experts && mid > 0 && shared > 0) ||
            experts > 65536 || mid > 0x7fffffff || shared > 0x7fffffff)
            return fail(HYQ_EINVAL, "invalid expert dimensions");
        if ((rc = integer("expert_gating_func", &gating))) return rc;
        if (gating != 2) return fail(HYQ_EINVAL, "HYV3 requires a sigmoid router");
        hyq_weight *router, *eg, *eu, *ed, *sg, *su, *sd;
        std::vector<float> bias;
        if ((rc = matrix(ctx, g, p + "ffn_gate_inp.weight", {H, experts}, own, &router)))
            return rc;
        if (router->dtype != HYQ_F32) return fail(HYQ_EINVAL, "HYV3 router must use F32");
        if ((rc = norm(ctx, g, p + "exp_probs_b", experts, bias)) ||
            (rc = real("expert_weights_scale", &scale)))
            return rc;
        if (!(scale > 0.f)) return fail(HYQ_EINVAL, "invalid expert weight scale");
        if ((rc = matrix(ctx, g, p + "ffn_gate_exps.weight", {H, mid, experts}, own, &eg)) ||
            (rc = matrix(ctx, g, p + "ffn_up_exps.weight", {H, mid, experts}, own, &eu)) ||
            (rc = matrix(ctx, g, p + "ffn_down_exps.weight", {mid, H, experts}, own, &ed)) ||
            (rc = matrix(ctx, g, p + "ffn_gate_shexp.weight", {H, shared}, own, &sg)) ||
            (rc = matrix(ctx, g, p + "ffn_up_shexp.weight", {H, shared}, own, &su)) ||
            (rc = matrix(ctx, g, p + "ffn_down_shexp.weight", {shared, H}, own, &sd)) ||
            (rc = hyq_gguf_meta_bool(g, (prefix + ".expert_weights_norm").c_str(), &norm_w)))
            return rc;
        hyq_moe_config mc{(int)experts, (int)used, (int)mid, (int)shared, norm_w, scale};
        if ((rc = hyq_dense_set_moe(m, (int)i, &mc, router, bias.data(), eg, eu, ed, sg, su,
                                    sd)))
            return rc;
    }
    if ((rc = hyq_dense_set_output(m, emb, outw, onorm.data()))) return rc;
    for (hyq_weight *w : own.w) dense_adopt(m, w);
    own.w.clear();
    *out = guard.release();
    return HYQ_OK;
}
