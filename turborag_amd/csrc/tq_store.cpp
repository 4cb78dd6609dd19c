// tq_store.cpp — the on-disk CAG store formats, host side.
//
// The reference writes, per (document, layer, scheme) (tq_backend/cag_store.py):
//   <key>.bin   turbo schemes: the raw page pool (:147-149); fp16: torch.save
//               of {"num_tokens", "kv", "shape"} (:128-131)
//   <key>.meta  torch.save({"num_tokens": N, "slots": int32[N]}) (:150)
//   manifest.json {"v": 1, "entries": {doc_id: {"sha256", "layers":
//               {"<layer>::<scheme>": {"key", "num_tokens", "stored_at"}}}}}
//               (:48-67), written to a .tmp file and renamed (:40-45)
// with key = sha256(doc_id)[:16] + "_L%02d_" + scheme (:97-100).
//
// Here those files are produced and consumed without Python:
//   * SHA-256 (FIPS 180-4) for the keys and manifest hashes;
//   * torch.save files: a zip archive of stored (uncompressed) records, the
//     pickle in <archive>/data.pkl and tensor storages in <archive>/data/<k>
//     (records 64-byte aligned, as torch writes them);
//   * a restricted pickle reader that builds values for the opcodes and the
//     three globals torch.save emits for dicts of ints, strings, lists and
//     tensors, and rejects everything else (no code runs while reading, unlike
//     the reference's torch.load(weights_only=False), :172);
//   * a versioned 64-byte footer after the raw pages of a .bin (the format is
//     otherwise unversioned): geometry, token count and a CRC-32C of the
//     pages.  The reference's reader slices raw[:pool_bytes] (:189-190), so it
//     ignores the footer, and footer-less files from the reference load here;
//   * the manifest, read and rewritten with Python's json.dumps(indent=2)
//     layout so that both implementations can share one store.
#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "tq_internal.h"

namespace tq {
namespace store {

// ---------------------------------------------------------------------------
// SHA-256 (FIPS 180-4 section 6.2)
// ---------------------------------------------------------------------------
namespace {
constexpr uint32_t kK256[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
    0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
    0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
    0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
    0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
    0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
    0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
    0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
    0xc67178f2};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

void sha256_block(uint32_t h[8], const uint8_t* p) {
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
        w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 |
               (uint32_t)p[4 * t + 2] << 8 | (uint32_t)p[4 * t + 3];
    for (int t = 16; t < 64; ++t) {
        const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
        const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
        w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int t = 0; t < 64; ++t) {
        const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
        const uint32_t ch = (e & f) ^ (~e & g);
        const uint32_t t1 = hh + S1 + ch + kK256[t] + w[t];
        const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
        const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
        const uint32_t t2 = S0 + maj;
        hh = g;
        g = f;
        f = e;
        e = d + t1;
        d = c;
        c = b;
        b = a;
        a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d;
    h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}
}  // namespace

std::string sha256_hex(const void* data, size_t n) {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                     0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    const uint8_t* p = static_cast<const uint8_t*>(data);
    size_t i = 0;
    for (; i + 64 <= n; i += 64) sha256_block(h, p + i);
    uint8_t tail[128] = {0};
    const size_t rem = n - i;
    if (rem) std::memcpy(tail, p + i, rem);
    tail[rem] = 0x80;
    const size_t tl = rem + 9 <= 64 ? 64 : 128;
    const uint64_t bits = (uint64_t)n * 8;
    for (int k = 0; k < 8; ++k) tail[tl - 1 - k] = (uint8_t)(bits >> (8 * k));
    sha256_block(h, tail);
    if (tl == 128) sha256_block(h, tail + 64);
    static const char* hex = "0123456789abcdef";
    std::string out(64, '0');
    for (int k = 0; k < 8; ++k)
        for (int b = 0; b < 8; ++b) out[8 * k + b] = hex[(h[k] >> (28 - 4 * b)) & 0xF];
    return out;
}

// ---------------------------------------------------------------------------
// CRC-32 (zip records: reflected polynomial 0xEDB88320) and CRC-32C (page
// footer: reflected Castagnoli polynomial 0x82F63B78; SSE4.2 crc32 when the
// host has it, 8 table lookups per 8 bytes otherwise).
// ---------------------------------------------------------------------------
namespace {
struct CrcTables {
    uint32_t zip[256];
    uint32_t c[8][256];
    CrcTables() {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t a = i, b = i;
            for (int k = 0; k < 8; ++k) {
                a = (a >> 1) ^ ((a & 1) ? 0xEDB88320u : 0u);
                b = (b >> 1) ^ ((b & 1) ? 0x82F63B78u : 0u);
            }
            zip[i] = a;
            c[0][i] = b;
        }
        for (int t = 1; t < 8; ++t)
            for (uint32_t i = 0; i < 256; ++i)
                c[t][i] = (c[t - 1][i] >> 8) ^ c[0][c[t - 1][i] & 0xFF];
    }
};
const CrcTables& crc_tables() {
    static const CrcTables t;
    return t;
}

__attribute__((target("sse4.2"))) uint32_t crc32c_hw(uint32_t crc, const uint8_t* p, size_t n) {
    uint64_t c = crc;
    for (; n >= 8; n -= 8, p += 8) {
        uint64_t v;
        std::memcpy(&v, p, 8);
        c = __builtin_ia32_crc32di(c, v);
    }
    uint32_t c32 = (uint32_t)c;
    for (; n; --n, ++p) c32 = __builtin_ia32_crc32qi(c32, *p);
    return c32;
}

uint32_t crc32c_sw(uint32_t crc, const uint8_t* p, size_t n) {
    const auto& T = crc_tables().c;
    for (; n >= 8; n -= 8, p += 8) {
        const uint32_t lo = crc ^ ((uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 |
                                   (uint32_t)p[3] << 24);
        crc = T[7][lo & 0xFF] ^ T[6][(lo >> 8) & 0xFF] ^ T[5][(lo >> 16) & 0xFF] ^
              T[4][lo >> 24] ^ T[3][p[4]] ^ T[2][p[5]] ^ T[1][p[6]] ^ T[0][p[7]];
    }
    for (; n; --n, ++p) crc = (crc >> 8) ^ T[0][(crc ^ *p) & 0xFF];
    return crc;
}
}  // namespace

uint32_t crc32_zip(const void* data, size_t n) {
    const auto& T = crc_tables().zip;
    uint32_t c = 0xFFFFFFFFu;
    const uint8_t* p = static_cast<const uint8_t*>(data);
    for (size_t i = 0; i < n; ++i) c = (c >> 8) ^ T[(c ^ p[i]) & 0xFF];
    return c ^ 0xFFFFFFFFu;
}

uint32_t crc32c(const void* data, size_t n) {
    static const bool hw = __builtin_cpu_supports("sse4.2");
    const uint8_t* p = static_cast<const uint8_t*>(data);
    return ~(hw ? crc32c_hw(0xFFFFFFFFu, p, n) : crc32c_sw(0xFFFFFFFFu, p, n));
}

uint32_t crc32c_portable(const void* data, size_t n) {
    return ~crc32c_sw(0xFFFFFFFFu, static_cast<const uint8_t*>(data), n);
}

// ---------------------------------------------------------------------------
// Files
// ---------------------------------------------------------------------------
namespace {
std::string read_file(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) throw Error("cannot open " + path);
    std::string s;
    char buf[1 << 16];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) s.append(buf, n);
    const bool bad = std::ferror(f);
    std::fclose(f);
    if (bad) throw Error("read error on " + path);
    return s;
}

// Writes to <path>.tmp, then renames it over path (a reader never sees a
// partial file; the reference writes its manifest the same way).
void write_file_atomic(const std::string& path, const std::vector<std::pair<const void*, size_t>>& parts) {
    const std::string tmp = path + ".tmp";
    FILE* f = std::fopen(tmp.c_str(), "wb");
    if (!f) throw Error("cannot create " + tmp);
    bool ok = true;
    for (const auto& p : parts)
        if (p.second && std::fwrite(p.first, 1, p.second, f) != p.second) ok = false;
    if (std::fclose(f) != 0) ok = false;
    if (!ok || std::rename(tmp.c_str(), path.c_str()) != 0) {
        std::remove(tmp.c_str());
        throw Error("write failed: " + path);
    }
}

void put16(std::string& s, uint16_t v) { s.append(reinterpret_cast<const char*>(&v), 2); }
void put32(std::string& s, uint32_t v) { s.append(reinterpret_cast<const char*>(&v), 4); }
void put64(std::string& s, uint64_t v) { s.append(reinterpret_cast<const char*>(&v), 8); }
// True when [o, o + n) lies inside a buffer of `size` bytes.  Written without
// o + n, which wraps for offsets read from a file.
bool in_bounds(uint64_t o, uint64_t n, uint64_t size) { return o <= size && n <= size - o; }
uint16_t get16(const std::string& s, uint64_t o) {
    if (!in_bounds(o, 2, s.size())) throw Error("zip: truncated");
    uint16_t v;
    std::memcpy(&v, s.data() + o, 2);
    return v;
}
uint32_t get32(const std::string& s, uint64_t o) {
    if (!in_bounds(o, 4, s.size())) throw Error("zip: truncated");
    uint32_t v;
    std::memcpy(&v, s.data() + o, 4);
    return v;
}
uint64_t get64(const std::string& s, uint64_t o) {
    if (!in_bounds(o, 8, s.size())) throw Error("zip: truncated");
    uint64_t v;
    std::memcpy(&v, s.data() + o, 8);
    return v;
}
}  // namespace

// ---------------------------------------------------------------------------
// Zip archives of stored records (APPNOTE 6.3: local headers, central
// directory, end record; zip64 records read when present).
// ---------------------------------------------------------------------------
struct ZipRecord {
    std::string name;
    size_t offset, size;
};

std::vector<ZipRecord> zip_records(const std::string& z) {
    if (z.size() < 22) throw Error("zip: file too short");
    size_t eocd = std::string::npos;
    const size_t lo = z.size() > 22 + 65535 ? z.size() - 22 - 65535 : 0;
    for (size_t i = z.size() - 22 + 1; i-- > lo;)
        if (get32(z, i) == 0x06054b50u) {
            eocd = i;
            break;
        }
    if (eocd == std::string::npos) throw Error("zip: no end of central directory");
    uint64_t count = get16(z, eocd + 10), cd_off = get32(z, eocd + 16);
    if ((count == 0xFFFF || cd_off == 0xFFFFFFFFu) && eocd >= 20 && get32(z, eocd - 20) == 0x07064b50u) {
        const uint64_t e64 = get64(z, eocd - 20 + 8);
        if (get32(z, e64) != 0x06064b50u) throw Error("zip: bad zip64 end record");
        count = get64(z, e64 + 32);
        cd_off = get64(z, e64 + 48);
    }
    // Every offset and size below comes from the file: each is checked against
    // the file's size before use (get16/32/64, in_bounds), never by a sum
    // that could wrap.
    if (cd_off > z.size()) throw Error("zip: central directory offset beyond the file");
    std::vector<ZipRecord> out;
    uint64_t p = cd_off;
    for (uint64_t k = 0; k < count; ++k) {
        if (get32(z, p) != 0x02014b50u) throw Error("zip: bad central directory entry");
        const uint16_t method = get16(z, p + 10);
        uint64_t csize = get32(z, p + 20), usize = get32(z, p + 24);
        const uint16_t nl = get16(z, p + 28), xl = get16(z, p + 30), cl = get16(z, p + 32);
        uint64_t lho = get32(z, p + 42);
        // p + 46 <= size (get32 at p + 42 passed), so these sums cannot wrap
        if (!in_bounds(p + 46, (uint64_t)nl + xl + cl, z.size()))
            throw Error("zip: truncated central directory entry");
        std::string name = z.substr(p + 46, nl);
        // zip64 extended information (id 1): the 0xFFFFFFFF fields, in order
        const uint64_t xend = p + 46 + nl + xl;
        for (uint64_t x = p + 46 + nl; x + 4 <= xend;) {
            const uint16_t id = get16(z, x), len = get16(z, x + 2);
            if (x + 4 + len > xend) throw Error("zip: extra field overruns its entry");
            if (id == 1) {
                uint64_t q = x + 4;
                const uint64_t qend = x + 4 + len;
                auto next64 = [&]() {
                    if (q + 8 > qend) throw Error("zip: short zip64 extra field");
                    const uint64_t v = get64(z, q);
                    q += 8;
                    return v;
                };
                if (usize == 0xFFFFFFFFu) usize = next64();
                if (csize == 0xFFFFFFFFu) csize = next64();
                if (lho == 0xFFFFFFFFu) lho = next64();
            }
            x += 4 + len;
        }
        if (method != 0 || csize != usize) throw Error("zip: record '" + name + "' is compressed");
        if (lho > z.size() || usize > z.size())
            throw Error("zip: record '" + name + "' offset or size beyond the file");
        if (get32(z, lho) != 0x04034b50u) throw Error("zip: bad local header");
        // lho + 30 <= size (get16 at lho + 28 passed); the two lengths are < 2^16
        const uint64_t data = lho + 30 + (uint64_t)get16(z, lho + 26) + get16(z, lho + 28);
        if (!in_bounds(data, usize, z.size())) throw Error("zip: record '" + name + "' truncated");
        out.push_back({name, (size_t)data, (size_t)usize});
        p += 46 + (uint64_t)nl + xl + cl;
    }
    return out;
}

// Writes records as torch.save does: stored, data 64-byte aligned through a
// padding extra field (id 0x4246 'FB'), CRC-32 and sizes in the headers.
std::string zip_archive(const std::vector<std::pair<std::string, std::string>>& recs) {
    std::string z, cd;
    for (const auto& r : recs) {
        const size_t lho = z.size();
        const uint32_t crc = crc32_zip(r.second.data(), r.second.size());
        const size_t base = lho + 30 + r.first.size();
        size_t pad = (64 - (base + 4) % 64) % 64;
        put32(z, 0x04034b50u);
        put16(z, 20);      // version needed
        put16(z, 0x0800);  // utf-8 names
        put16(z, 0);       // stored
        put16(z, 0);
        put16(z, 0x21);    // DOS date 1980-01-01
        put32(z, crc);
        put32(z, (uint32_t)r.second.size());
        put32(z, (uint32_t)r.second.size());
        put16(z, (uint16_t)r.first.size());
        put16(z, (uint16_t)(4 + pad));
        z += r.first;
        put16(z, 0x4246);
        put16(z, (uint16_t)pad);
        z.append(pad, 'Z');
        z += r.second;
        put32(cd, 0x02014b50u);
        put16(cd, 20);
        put16(cd, 20);
        put16(cd, 0x0800);
        put16(cd, 0);
        put16(cd, 0);
        put16(cd, 0x21);
        put32(cd, crc);
        put32(cd, (uint32_t)r.second.size());
        put32(cd, (uint32_t)r.second.size());
        put16(cd, (uint16_t)r.first.size());
        put16(cd, 0);
        put16(cd, 0);
        put16(cd, 0);
        put16(cd, 0);
        put32(cd, 0);
        put32(cd, (uint32_t)lho);
        cd += r.first;
    }
    const size_t cd_off = z.size();
    z += cd;
    put32(z, 0x06054b50u);
    put16(z, 0);
    put16(z, 0);
    put16(z, (uint16_t)recs.size());
    put16(z, (uint16_t)recs.size());
    put32(z, (uint32_t)cd.size());
    put32(z, (uint32_t)cd_off);
    put16(z, 0);
    return z;
}

// ---------------------------------------------------------------------------
// Pickle values: the subset torch.save emits for {str: int | str | list |
// tensor} (protocol 2, with the later framing opcodes accepted).
// ---------------------------------------------------------------------------
struct Value;
using VP = std::shared_ptr<Value>;
struct Value {
    enum Kind { None, Bool, Int, Float, Str, List, Tuple, Dict, Global, Storage, Tensor, Mark } kind;
    int64_t i = 0;
    double f = 0;
    std::string s;                            // Str; Global "module.name"; Storage dtype name
    std::vector<VP> items;                    // List, Tuple
    std::vector<std::pair<VP, VP>> dict;      // Dict (insertion order)
    std::string key;                          // Storage / Tensor: record key under data/
    int64_t numel = 0, offset = 0;            // Storage numel; Tensor storage offset
    std::vector<int64_t> shape, stride;       // Tensor
    explicit Value(Kind k) : kind(k) {}
};

namespace {
VP mk(Value::Kind k) { return std::make_shared<Value>(k); }
VP mk_int(int64_t v) { auto p = mk(Value::Int); p->i = v; return p; }
VP mk_str(std::string v) { auto p = mk(Value::Str); p->s = std::move(v); return p; }

std::vector<int64_t> int_tuple(const VP& v) {
    if (v->kind != Value::Tuple) throw Error("pickle: expected a tuple of ints");
    std::vector<int64_t> out;
    for (const auto& x : v->items) {
        if (x->kind != Value::Int) throw Error("pickle: expected a tuple of ints");
        out.push_back(x->i);
    }
    return out;
}

// Element size of the storage types torch.save names.
int storage_elem_bytes(const std::string& t) {
    static const std::map<std::string, int> m = {
        {"ByteStorage", 1}, {"CharStorage", 1}, {"BoolStorage", 1}, {"ShortStorage", 2},
        {"HalfStorage", 2}, {"BFloat16Storage", 2}, {"IntStorage", 4}, {"FloatStorage", 4},
        {"LongStorage", 8}, {"DoubleStorage", 8}};
    auto it = m.find(t);
    return it == m.end() ? 0 : it->second;
}
}  // namespace

VP unpickle(const std::string& b) {
    std::vector<VP> st;
    std::vector<size_t> marks;
    std::map<int64_t, VP> memo;
    size_t p = 0;
    // p <= b.size() always holds, so b.size() - p cannot wrap; n comes from
    // the file (up to 2^64 - 1 for BINUNICODE8) and is never added to p
    // before this check.
    auto need = [&](uint64_t n) {
        if (n > b.size() - p) throw Error("pickle: truncated");
    };
    auto u8 = [&]() { need(1); return (uint8_t)b[p++]; };
    auto u16 = [&]() { need(2); uint16_t v; std::memcpy(&v, b.data() + p, 2); p += 2; return v; };
    auto u32 = [&]() { need(4); uint32_t v; std::memcpy(&v, b.data() + p, 4); p += 4; return v; };
    auto bytes = [&](uint64_t n) { need(n); std::string s = b.substr(p, n); p += n; return s; };
    auto line = [&]() {
        const size_t e = b.find('\n', p);
        if (e == std::string::npos) throw Error("pickle: truncated");
        std::string s = b.substr(p, e - p);
        p = e + 1;
        return s;
    };
    auto pop = [&]() {
        if (st.empty()) throw Error("pickle: stack underflow");
        VP v = st.back();
        st.pop_back();
        return v;
    };
    auto pop_mark = [&]() {
        if (marks.empty() || marks.back() > st.size()) throw Error("pickle: no mark");
        const size_t m = marks.back();
        marks.pop_back();
        std::vector<VP> items(st.begin() + m, st.end());
        st.resize(m);
        return items;
    };
    auto global = [&](const std::string& mod, const std::string& name) {
        const std::string full = mod + "." + name;
        const bool ok = full == "torch._utils._rebuild_tensor_v2" ||
                        full == "collections.OrderedDict" ||
                        (mod == "torch" && storage_elem_bytes(name) > 0);
        if (!ok) throw Error("pickle: global '" + full + "' is not allowed");
        auto g = mk(Value::Global);
        g->s = full;
        st.push_back(g);
    };
    auto set_items = [&](VP d, const std::vector<VP>& kv) {
        if (d->kind != Value::Dict || kv.size() % 2) throw Error("pickle: bad SETITEMS");
        for (size_t k = 0; k < kv.size(); k += 2) d->dict.emplace_back(kv[k], kv[k + 1]);
    };
    for (;;) {
        const uint8_t op = u8();
        switch (op) {
            case 0x80: u8(); break;                   // PROTO
            case 0x95: need(8); p += 8; break;         // FRAME
            case '}': st.push_back(mk(Value::Dict)); break;
            case ']': st.push_back(mk(Value::List)); break;
            case ')': st.push_back(mk(Value::Tuple)); break;
            case '(': marks.push_back(st.size()); break;
            case 'N': st.push_back(mk(Value::None)); break;
            case 0x88: case 0x89: {
                auto v = mk(Value::Bool);
                v->i = op == 0x88;
                st.push_back(v);
                break;
            }
            case 'K': st.push_back(mk_int(u8())); break;
            case 'M': st.push_back(mk_int(u16())); break;
            case 'J': st.push_back(mk_int((int32_t)u32())); break;
            case 0x8a: {  // LONG1: little-endian two's complement
                const uint8_t n = u8();
                if (n > 8) throw Error("pickle: integer too large");
                const std::string s = bytes(n);
                uint64_t v = 0;
                for (int k = n - 1; k >= 0; --k) v = (v << 8) | (uint8_t)s[k];
                if (n && n < 8 && (s[n - 1] & 0x80)) v |= ~0ull << (8 * n);
                st.push_back(mk_int((int64_t)v));
                break;
            }
            case 'G': {
                need(8);
                uint64_t v = 0;
                for (int k = 0; k < 8; ++k) v = (v << 8) | (uint8_t)b[p + k];
                p += 8;
                auto x = mk(Value::Float);
                std::memcpy(&x->f, &v, 8);
                st.push_back(x);
                break;
            }
            case 'X': st.push_back(mk_str(bytes(u32()))); break;
            case 0x8c: st.push_back(mk_str(bytes(u8()))); break;
            case 0x8d: {
                need(8);
                uint64_t n;
                std::memcpy(&n, b.data() + p, 8);
                p += 8;
                st.push_back(mk_str(bytes(n)));
                break;
            }
            case 't': {
                auto t = mk(Value::Tuple);
                t->items = pop_mark();
                st.push_back(t);
                break;
            }
            case 0x85: case 0x86: case 0x87: {
                const int n = op - 0x84;
                auto t = mk(Value::Tuple);
                t->items.resize(n);
                for (int k = n - 1; k >= 0; --k) t->items[k] = pop();
                st.push_back(t);
                break;
            }
            case 'q': if (st.empty()) throw Error("pickle: empty stack"); memo[u8()] = st.back(); break;
            case 'r': if (st.empty()) throw Error("pickle: empty stack"); memo[u32()] = st.back(); break;
            case 0x94: if (st.empty()) throw Error("pickle: empty stack"); memo[(int64_t)memo.size()] = st.back(); break;
            case 'h': case 'j': {
                const int64_t k = op == 'h' ? u8() : u32();
                auto it = memo.find(k);
                if (it == memo.end()) throw Error("pickle: bad memo reference");
                st.push_back(it->second);
                break;
            }
            case 'c': {
                const std::string mod = line();
                const std::string name = line();
                global(mod, name);
                break;
            }
            case 0x93: {  // STACK_GLOBAL
                VP name = pop(), mod = pop();
                if (mod->kind != Value::Str || name->kind != Value::Str) throw Error("pickle: bad STACK_GLOBAL");
                global(mod->s, name->s);
                break;
            }
            case 'Q': {  // BINPERSID: ('storage', StorageType, key, location, numel)
                VP pid = pop();
                if (pid->kind != Value::Tuple || pid->items.size() < 5 ||
                    pid->items[0]->kind != Value::Str || pid->items[0]->s != "storage" ||
                    pid->items[1]->kind != Value::Global || pid->items[2]->kind != Value::Str ||
                    pid->items[4]->kind != Value::Int)
                    throw Error("pickle: unsupported persistent id");
                auto s = mk(Value::Storage);
                s->s = pid->items[1]->s.substr(pid->items[1]->s.rfind('.') + 1);
                s->key = pid->items[2]->s;
                s->numel = pid->items[4]->i;
                st.push_back(s);
                break;
            }
            case 'R': {
                VP args = pop(), fn = pop();
                if (fn->kind != Value::Global || args->kind != Value::Tuple) throw Error("pickle: bad REDUCE");
                if (fn->s == "collections.OrderedDict") {
                    if (!args->items.empty()) throw Error("pickle: OrderedDict with arguments");
                    st.push_back(mk(Value::Dict));
                } else if (fn->s == "torch._utils._rebuild_tensor_v2") {
                    if (args->items.size() < 4 || args->items[0]->kind != Value::Storage ||
                        args->items[1]->kind != Value::Int)
                        throw Error("pickle: bad _rebuild_tensor_v2 arguments");
                    auto t = mk(Value::Tensor);
                    t->s = args->items[0]->s;
                    t->key = args->items[0]->key;
                    t->numel = args->items[0]->numel;
                    t->offset = args->items[1]->i;
                    t->shape = int_tuple(args->items[2]);
                    t->stride = int_tuple(args->items[3]);
                    st.push_back(t);
                } else {
                    throw Error("pickle: call of '" + fn->s + "' is not allowed");
                }
                break;
            }
            case 's': {
                VP v = pop(), k = pop();
                if (st.empty()) throw Error("pickle: bad SETITEM");
                set_items(st.back(), {k, v});
                break;
            }
            case 'u': {
                auto kv = pop_mark();
                if (st.empty()) throw Error("pickle: bad SETITEMS");
                set_items(st.back(), kv);
                break;
            }
            case 'a': {
                VP v = pop();
                if (st.empty() || st.back()->kind != Value::List) throw Error("pickle: bad APPEND");
                st.back()->items.push_back(v);
                break;
            }
            case 'e': {
                auto items = pop_mark();
                if (st.empty() || st.back()->kind != Value::List) throw Error("pickle: bad APPENDS");
                for (auto& v : items) st.back()->items.push_back(v);
                break;
            }
            case '.':
                if (st.size() != 1) throw Error("pickle: stack not empty at STOP");
                return st.back();
            default: {
                char msg[64];
                std::snprintf(msg, sizeof(msg), "pickle: opcode 0x%02x is not allowed", op);
                throw Error(msg);
            }
        }
    }
}

namespace {
// Pickle writer (protocol 2), no memo: what torch.load needs for
// {str: int | str | list[int] | tensor} with one storage per tensor.
struct Pickler {
    std::string b;
    void op(char c) { b += c; }
    void str(const std::string& s) {
        op('X');
        put32(b, (uint32_t)s.size());
        b += s;
    }
    void integer(int64_t v) {
        if (v >= 0 && v < 256) {
            op('K');
            b += (char)v;
        } else if (v >= 0 && v < 65536) {
            op('M');
            put16(b, (uint16_t)v);
        } else if (v >= INT32_MIN && v <= INT32_MAX) {
            op('J');
            put32(b, (uint32_t)(int32_t)v);
        } else {
            b += (char)0x8a;
            b += (char)8;
            put64(b, (uint64_t)v);
        }
    }
    void global(const char* mod, const char* name) {
        op('c');
        b += mod;
        b += '\n';
        b += name;
        b += '\n';
    }
    // torch._utils._rebuild_tensor_v2(storage, 0, shape, stride, False, OrderedDict())
    void tensor(const char* storage_type, const std::string& key, int64_t numel,
                const std::vector<int64_t>& shape) {
        global("torch._utils", "_rebuild_tensor_v2");
        op('(');
        op('(');
        str("storage");
        global("torch", storage_type);
        str(key);
        str("cpu");
        integer(numel);
        op('t');
        op('Q');
        integer(0);
        std::vector<int64_t> stride(shape.size(), 1);
        for (int k = (int)shape.size() - 2; k >= 0; --k) stride[k] = stride[k + 1] * shape[k + 1];
        op('(');
        for (auto v : shape) integer(v);
        op('t');
        op('(');
        for (auto v : stride) integer(v);
        op('t');
        b += (char)0x89;  // requires_grad False
        global("collections", "OrderedDict");
        op(')');
        op('R');
        op('t');
        op('R');
    }
};

// The archive name torch.save uses: the file's base name without extension.
std::string archive_name(const std::string& path) {
    std::string base = path.substr(path.find_last_of('/') + 1);
    const size_t dot = base.find('.');
    if (dot != std::string::npos && dot > 0) base = base.substr(0, dot);
    return base.empty() ? "archive" : base;
}

struct TorchFile {
    VP root;
    std::string blob;                    // whole file
    std::map<std::string, ZipRecord> data;  // storage key -> record
};

TorchFile torch_load(const std::string& path) {
    TorchFile t;
    t.blob = read_file(path);
    const ZipRecord* pkl = nullptr;
    auto recs = zip_records(t.blob);
    for (const auto& r : recs) {
        const size_t slash = r.name.find('/');
        const std::string rel = slash == std::string::npos ? r.name : r.name.substr(slash + 1);
        if (rel == "data.pkl") pkl = &r;
        if (rel.rfind("data/", 0) == 0) t.data[rel.substr(5)] = r;
    }
    if (!pkl) throw Error(path + ": not a torch.save archive (no data.pkl)");
    t.root = unpickle(t.blob.substr(pkl->offset, pkl->size));
    if (t.root->kind != Value::Dict) throw Error(path + ": top-level object is not a dict");
    return t;
}

VP dict_get(const VP& d, const std::string& k) {
    for (const auto& kv : d->dict)
        if (kv.first->kind == Value::Str && kv.first->s == k) return kv.second;
    return nullptr;
}

// Contiguous elements of a tensor value (C order over its storage).
const char* tensor_data(const TorchFile& t, const VP& v, const char* want_type, int64_t* numel) {
    if (!v || v->kind != Value::Tensor) throw Error("expected a tensor");
    if (v->s != want_type) throw Error(std::string("expected a ") + want_type + " tensor, got " + v->s);
    if (v->shape.size() != v->stride.size()) throw Error("tensor shape and stride ranks differ");
    auto it = t.data.find(v->key);
    if (it == t.data.end()) throw Error("tensor storage record missing");
    const int eb = storage_elem_bytes(v->s);
    // Elements the storage record holds; shape, stride and offset come from
    // the file and are checked against it without overflowing.
    const uint64_t cap = it->second.size / (uint64_t)eb;
    uint64_t n = 1, expect = 1;
    for (int k = (int)v->shape.size() - 1; k >= 0; --k) {
        if (v->shape[k] < 0) throw Error("tensor has a negative dimension");
        const uint64_t d = (uint64_t)v->shape[k];
        if (d != 1 && (uint64_t)v->stride[k] != expect) throw Error("tensor is not contiguous");
        if (d != 0 && n > cap / d) throw Error("tensor exceeds its storage");
        n *= d;
        expect = n;
    }
    if (v->offset < 0 || (uint64_t)v->offset > cap || n > cap - (uint64_t)v->offset)
        throw Error("tensor exceeds its storage");
    *numel = (int64_t)n;
    return t.blob.data() + it->second.offset + (size_t)v->offset * eb;
}

std::string torch_archive(const std::string& path, const std::string& pkl,
                          const std::vector<std::string>& storages) {
    const std::string a = archive_name(path);
    std::vector<std::pair<std::string, std::string>> recs;
    recs.emplace_back(a + "/data.pkl", pkl);
    recs.emplace_back(a + "/.format_version", "1");
    recs.emplace_back(a + "/.storage_alignment", "64");
    recs.emplace_back(a + "/byteorder", "little");
    for (size_t k = 0; k < storages.size(); ++k)
        recs.emplace_back(a + "/data/" + std::to_string(k), storages[k]);
    recs.emplace_back(a + "/version", "3\n");
    // torch writes a random 40-digit id; a content hash serves the same purpose
    std::string id = sha256_hex(pkl.data(), pkl.size());
    std::string digits;
    for (char c : id) digits += (char)('0' + (c % 10));
    recs.emplace_back(a + "/.data/serialization_id", digits.substr(0, 40));
    return zip_archive(recs);
}
}  // namespace

// ---------------------------------------------------------------------------
// .meta and fp16 .bin
// ---------------------------------------------------------------------------
void write_meta(const std::string& path, int64_t num_tokens, const int32_t* slots, int64_t n,
                const TQStoreFormat* fmt) {
    Pickler pk;
    pk.b += (char)0x80;
    pk.b += (char)2;
    pk.op('}');
    pk.op('(');
    pk.str("num_tokens");
    pk.integer(num_tokens);
    pk.str("slots");
    pk.tensor("IntStorage", "0", n, {n});
    if (fmt) {  // the format record (extra keys; the reference reads only the two above)
        const std::pair<const char*, int64_t> kv[] = {
            {"tq_format", fmt->version}, {"tq_scheme", fmt->scheme},
            {"num_kv_heads", fmt->num_kv_heads}, {"head_dim", fmt->head_dim},
            {"block_size", fmt->block_size}, {"page_size_bytes", fmt->page_size_bytes}};
        for (const auto& e : kv) {
            pk.str(e.first);
            pk.integer(e.second);
        }
    }
    pk.op('u');
    pk.op('.');
    const std::string z = torch_archive(path, pk.b, {std::string(reinterpret_cast<const char*>(slots), n * 4)});
    write_file_atomic(path, {{z.data(), z.size()}});
}

bool read_meta(const std::string& path, int64_t* num_tokens, std::vector<int32_t>* slots,
               TQStoreFormat* fmt) {
    const TorchFile t = torch_load(path);
    VP nt = dict_get(t.root, "num_tokens");
    if (!nt || nt->kind != Value::Int) throw Error(path + ": no integer 'num_tokens'");
    *num_tokens = nt->i;
    int64_t n = 0;
    const char* d = tensor_data(t, dict_get(t.root, "slots"), "IntStorage", &n);
    slots->resize(n);
    if (n) std::memcpy(slots->data(), d, n * 4);
    VP ver = dict_get(t.root, "tq_format");
    if (!ver || ver->kind != Value::Int) return false;
    if (fmt) {
        auto geti = [&](const char* k) {
            VP v = dict_get(t.root, k);
            if (!v || v->kind != Value::Int) throw Error(path + ": format record lacks " + k);
            return v->i;
        };
        std::memset(fmt, 0, sizeof(*fmt));
        fmt->version = (int32_t)ver->i;
        fmt->scheme = (int32_t)geti("tq_scheme");
        fmt->num_kv_heads = (int32_t)geti("num_kv_heads");
        fmt->head_dim = (int32_t)geti("head_dim");
        fmt->block_size = (int32_t)geti("block_size");
        fmt->page_size_bytes = (int32_t)geti("page_size_bytes");
        fmt->num_tokens = *num_tokens;
    }
    return true;
}

void write_fp16(const std::string& path, int64_t num_tokens, const uint16_t* kv, int64_t numel,
                const std::vector<int64_t>& shape) {
    Pickler pk;
    pk.b += (char)0x80;
    pk.b += (char)2;
    pk.op('}');
    pk.op('(');
    pk.str("num_tokens");
    pk.integer(num_tokens);
    pk.str("kv");
    pk.tensor("HalfStorage", "0", numel, {numel});
    pk.str("shape");
    pk.op(']');
    pk.op('(');
    for (auto v : shape) pk.integer(v);
    pk.op('e');
    pk.op('u');
    pk.op('.');
    const std::string z = torch_archive(path, pk.b, {std::string(reinterpret_cast<const char*>(kv), numel * 2)});
    write_file_atomic(path, {{z.data(), z.size()}});
}

void read_fp16(const std::string& path, int64_t* num_tokens, std::vector<uint16_t>* kv,
               std::vector<int64_t>* shape) {
    const TorchFile t = torch_load(path);
    VP nt = dict_get(t.root, "num_tokens");
    if (!nt || nt->kind != Value::Int) throw Error(path + ": no integer 'num_tokens'");
    *num_tokens = nt->i;
    int64_t n = 0;
    const char* d = tensor_data(t, dict_get(t.root, "kv"), "HalfStorage", &n);
    kv->resize(n);
    if (n) std::memcpy(kv->data(), d, n * 2);
    shape->clear();
    VP sh = dict_get(t.root, "shape");
    if (sh && sh->kind == Value::List)
        for (const auto& x : sh->items) {
            if (x->kind != Value::Int) throw Error(path + ": 'shape' is not a list of ints");
            shape->push_back(x->i);
        }
}

// ---------------------------------------------------------------------------
// .bin pages + footer
// ---------------------------------------------------------------------------
namespace {
struct Footer {  // 64 bytes, little-endian, after the pages
    char magic[8];
    uint32_t version, scheme;
    int32_t num_kv_heads, head_dim, block_size, page_size_bytes;
    uint64_t num_pages, num_tokens, pool_bytes;
    uint32_t crc32c, footer_bytes;
};
static_assert(sizeof(Footer) == 64, "footer layout");
constexpr char kMagic[8] = {'T', 'Q', 'P', 'A', 'G', 'E', 'S', '\0'};
}  // namespace

void write_pool(const std::string& path, const uint8_t* pool, size_t bytes, const TQStoreFormat& fmt) {
    Footer f;
    std::memset(&f, 0, sizeof(f));
    std::memcpy(f.magic, kMagic, 8);
    f.version = (uint32_t)fmt.version;
    f.scheme = (uint32_t)fmt.scheme;
    f.num_kv_heads = fmt.num_kv_heads;
    f.head_dim = fmt.head_dim;
    f.block_size = fmt.block_size;
    f.page_size_bytes = fmt.page_size_bytes;
    f.num_pages = (uint64_t)fmt.num_pages;
    f.num_tokens = (uint64_t)fmt.num_tokens;
    f.pool_bytes = bytes;
    f.crc32c = crc32c(pool, bytes);
    f.footer_bytes = sizeof(Footer);
    write_file_atomic(path, {{pool, bytes}, {&f, sizeof(f)}});
}

// Footer of a .bin if it has one; *file_bytes = size of the file.
bool pool_info(const std::string& path, size_t* file_bytes, TQStoreFormat* fmt, uint32_t* crc) {
    struct stat sb;
    if (stat(path.c_str(), &sb) != 0) throw Error("cannot stat " + path);
    *file_bytes = (size_t)sb.st_size;
    if (*file_bytes < sizeof(Footer)) return false;
    FILE* fp = std::fopen(path.c_str(), "rb");
    if (!fp) throw Error("cannot open " + path);
    Footer f;
    const bool got = std::fseek(fp, -(long)sizeof(Footer), SEEK_END) == 0 &&
                     std::fread(&f, 1, sizeof(f), fp) == sizeof(f);
    std::fclose(fp);
    if (!got || std::memcmp(f.magic, kMagic, 8) != 0 || f.footer_bytes != sizeof(Footer) ||
        f.pool_bytes != *file_bytes - sizeof(Footer))
        return false;
    if (fmt) {
        fmt->version = (int32_t)f.version;
        fmt->scheme = (int32_t)f.scheme;
        fmt->num_kv_heads = f.num_kv_heads;
        fmt->head_dim = f.head_dim;
        fmt->block_size = f.block_size;
        fmt->page_size_bytes = f.page_size_bytes;
        fmt->num_pages = (int64_t)f.num_pages;
        fmt->num_tokens = (int64_t)f.num_tokens;
    }
    if (crc) *crc = f.crc32c;
    return true;
}

// Reads the first `bytes` bytes of each file into dsts[k] (e.g. pinned host
// memory), files spread over `threads` threads.  With verify, files with a
// footer have their page checksum checked.
void read_pools(const char* const* paths, uint8_t* const* dsts, size_t bytes, int n, int threads,
                bool verify) {
    std::atomic<int> next{0};
    std::vector<std::string> errors(n);
    auto work = [&]() {
        for (int k; (k = next.fetch_add(1)) < n;) {
            try {
                const int fd = ::open(paths[k], O_RDONLY);
                if (fd < 0) throw Error(std::string("cannot open ") + paths[k]);
                size_t got = 0;
                while (got < bytes) {
                    const ssize_t r = ::pread(fd, dsts[k] + got, bytes - got, (off_t)got);
                    if (r <= 0) break;
                    got += (size_t)r;
                }
                ::close(fd);
                if (got < bytes)
                    throw Error(std::string(paths[k]) + ": shorter than the pool (" +
                                std::to_string(got) + " < " + std::to_string(bytes) + " bytes)");
                if (verify) {
                    size_t fb;
                    uint32_t crc;
                    if (pool_info(paths[k], &fb, nullptr, &crc) && fb == bytes + sizeof(Footer) &&
                        crc32c(dsts[k], bytes) != crc)
                        throw Error(std::string(paths[k]) + ": page checksum mismatch");
                }
            } catch (const std::exception& e) {
                errors[k] = e.what();
            }
        }
    };
    const int t = std::max(1, std::min(threads, n));
    std::vector<std::thread> pool;
    for (int i = 1; i < t; ++i) pool.emplace_back(work);
    work();
    for (auto& th : pool) th.join();
    for (const auto& e : errors)
        if (!e.empty()) throw Error(e);
}

// ---------------------------------------------------------------------------
// Manifest JSON (RFC 8259 values; written like Python's json.dumps(indent=2)
// with ensure_ascii, numbers kept as their original text).
// ---------------------------------------------------------------------------
struct Json {
    enum Kind { Null, True, False, Num, Str, Arr, Obj } kind = Null;
    std::string s;  // Num: literal text; Str: utf-8
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    Json* get(const std::string& k) {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
    Json& set(const std::string& k, Json v) {
        if (Json* j = get(k)) return *j = std::move(v);
        obj.emplace_back(k, std::move(v));
        return obj.back().second;
    }
    static Json str(const std::string& v) { Json j; j.kind = Str; j.s = v; return j; }
    static Json num(const std::string& v) { Json j; j.kind = Num; j.s = v; return j; }
    static Json object() { Json j; j.kind = Obj; return j; }
};

namespace {
struct JsonParser {
    const std::string& t;
    size_t p = 0;
    void ws() { while (p < t.size() && (t[p] == ' ' || t[p] == '\n' || t[p] == '\r' || t[p] == '\t')) ++p; }
    [[noreturn]] void fail() { throw Error("manifest: invalid JSON at byte " + std::to_string(p)); }
    void utf8(std::string& o, uint32_t c) {
        if (c < 0x80) o += (char)c;
        else if (c < 0x800) { o += (char)(0xC0 | c >> 6); o += (char)(0x80 | (c & 0x3F)); }
        else if (c < 0x10000) { o += (char)(0xE0 | c >> 12); o += (char)(0x80 | ((c >> 6) & 0x3F)); o += (char)(0x80 | (c & 0x3F)); }
        else { o += (char)(0xF0 | c >> 18); o += (char)(0x80 | ((c >> 12) & 0x3F)); o += (char)(0x80 | ((c >> 6) & 0x3F)); o += (char)(0x80 | (c & 0x3F)); }
    }
    uint32_t hex4() {
        if (p + 4 > t.size()) fail();
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = t[p++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else fail();
        }
        return v;
    }
    std::string string() {
        if (t[p] != '"') fail();
        ++p;
        std::string o;
        while (p < t.size() && t[p] != '"') {
            char c = t[p++];
            if (c != '\\') { o += c; continue; }
            if (p >= t.size()) fail();
            c = t[p++];
            switch (c) {
                case '"': o += '"'; break;
                case '\\': o += '\\'; break;
                case '/': o += '/'; break;
                case 'b': o += '\b'; break;
                case 'f': o += '\f'; break;
                case 'n': o += '\n'; break;
                case 'r': o += '\r'; break;
                case 't': o += '\t'; break;
                case 'u': {
                    uint32_t c1 = hex4();
                    if (c1 >= 0xD800 && c1 < 0xDC00 && p + 6 <= t.size() && t[p] == '\\' && t[p + 1] == 'u') {
                        p += 2;
                        const uint32_t c2 = hex4();
                        c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
                    }
                    utf8(o, c1);
                    break;
                }
                default: fail();
            }
        }
        if (p >= t.size()) fail();
        ++p;
        return o;
    }
    int depth = 0;  // nesting of the value being parsed (bounded: no deep recursion)
    Json value() {
        ws();
        if (p >= t.size()) fail();
        Json j;
        const char c = t[p];
        if ((c == '{' || c == '[') && depth >= 64) fail();
        struct Nest {
            int& d;
            explicit Nest(int& x) : d(x) { ++d; }
            ~Nest() { --d; }
        } nest(depth);
        if (c == '{') {
            j.kind = Json::Obj;
            ++p;
            ws();
            if (p < t.size() && t[p] == '}') { ++p; return j; }
            for (;;) {
                ws();
                std::string k = string();
                ws();
                if (p >= t.size() || t[p] != ':') fail();
                ++p;
                j.obj.emplace_back(std::move(k), value());
                ws();
                if (p < t.size() && t[p] == ',') { ++p; continue; }
                if (p < t.size() && t[p] == '}') { ++p; return j; }
                fail();
            }
        }
        if (c == '[') {
            j.kind = Json::Arr;
            ++p;
            ws();
            if (p < t.size() && t[p] == ']') { ++p; return j; }
            for (;;) {
                j.arr.push_back(value());
                ws();
                if (p < t.size() && t[p] == ',') { ++p; continue; }
                if (p < t.size() && t[p] == ']') { ++p; return j; }
                fail();
            }
        }
        if (c == '"') { j.kind = Json::Str; j.s = string(); return j; }
        if (t.compare(p, 4, "true") == 0) { p += 4; j.kind = Json::True; return j; }
        if (t.compare(p, 5, "false") == 0) { p += 5; j.kind = Json::False; return j; }
        if (t.compare(p, 4, "null") == 0) { p += 4; j.kind = Json::Null; return j; }
        const size_t b = p;
        while (p < t.size() && (std::isdigit((unsigned char)t[p]) || t[p] == '-' || t[p] == '+' ||
                                t[p] == '.' || t[p] == 'e' || t[p] == 'E'))
            ++p;
        if (p == b) fail();
        j.kind = Json::Num;
        j.s = t.substr(b, p - b);
        return j;
    }
};

void json_string(std::string& o, const std::string& s) {
    // json.dumps(ensure_ascii=True): the two-character escapes, and \uXXXX
    // (surrogate pairs above U+FFFF) for everything outside ' ' .. '~'.
    o += '"';
    for (size_t i = 0; i < s.size();) {
        const unsigned char c = (unsigned char)s[i];
        uint32_t cp = c;
        int len = 1;
        if (c >= 0xC0) {  // utf-8 lead byte
            len = c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : 2;
            cp = c & (0x7F >> len);
            for (int k = 1; k < len && i + k < s.size(); ++k) cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        i += len;
        char buf[16];
        switch (cp) {
            case '"': o += "\\\""; continue;
            case '\\': o += "\\\\"; continue;
            case '\n': o += "\\n"; continue;
            case '\r': o += "\\r"; continue;
            case '\t': o += "\\t"; continue;
            case '\b': o += "\\b"; continue;
            case '\f': o += "\\f"; continue;
            default: break;
        }
        if (cp >= 0x20 && cp < 0x7F) {
            o += (char)cp;
        } else if (cp < 0x10000) {
            std::snprintf(buf, sizeof(buf), "\\u%04x", cp);
            o += buf;
        } else {
            cp -= 0x10000;
            std::snprintf(buf, sizeof(buf), "\\u%04x\\u%04x", 0xD800 + (cp >> 10), 0xDC00 + (cp & 0x3FF));
            o += buf;
        }
    }
    o += '"';
}

void json_dump(std::string& o, const Json& j, int indent) {
    const std::string pad(indent + 2, ' '), end(indent, ' ');
    switch (j.kind) {
        case Json::Null: o += "null"; break;
        case Json::True: o += "true"; break;
        case Json::False: o += "false"; break;
        case Json::Num: o += j.s; break;
        case Json::Str: json_string(o, j.s); break;
        case Json::Arr:
            if (j.arr.empty()) { o += "[]"; break; }
            o += "[\n";
            for (size_t k = 0; k < j.arr.size(); ++k) {
                o += pad;
                json_dump(o, j.arr[k], indent + 2);
                o += k + 1 < j.arr.size() ? ",\n" : "\n";
            }
            o += end + "]";
            break;
        case Json::Obj:
            if (j.obj.empty()) { o += "{}"; break; }
            o += "{\n";
            for (size_t k = 0; k < j.obj.size(); ++k) {
                o += pad;
                json_string(o, j.obj[k].first);
                o += ": ";
                json_dump(o, j.obj[k].second, indent + 2);
                o += k + 1 < j.obj.size() ? ",\n" : "\n";
            }
            o += end + "}";
            break;
    }
}

// Python's repr of a float: the shortest decimal that reads back exactly.
std::string float_repr(double v) {
    char buf[40];
    for (int prec = 1; prec <= 17; ++prec) {
        std::snprintf(buf, sizeof(buf), "%.*g", prec, v);
        if (std::strtod(buf, nullptr) == v) break;
    }
    std::string s = buf;
    const size_t e = s.find('e');
    if (e != std::string::npos) {  // 1e+16 -> 1e+16 (Python keeps sign, 2+ digits)
        std::string mant = s.substr(0, e), ex = s.substr(e + 1);
        const char sign = ex[0] == '-' ? '-' : '+';
        if (ex[0] == '+' || ex[0] == '-') ex = ex.substr(1);
        while (ex.size() > 2 && ex[0] == '0') ex = ex.substr(1);
        return mant + "e" + sign + ex;
    }
    if (s.find('.') == std::string::npos && s.find("inf") == std::string::npos &&
        s.find("nan") == std::string::npos)
        s += ".0";
    return s;
}

std::string manifest_path(const std::string& dir) { return dir + "/manifest.json"; }

Json load_manifest(const std::string& dir) {
    Json m;
    try {
        const std::string text = read_file(manifest_path(dir));
        JsonParser jp{text};
        m = jp.value();
        if (m.kind != Json::Obj) throw Error("manifest: not an object");
    } catch (const Error&) {  // missing or unreadable: a fresh manifest (cag_store.py:33-38)
        m = Json::object();
        m.set("v", Json::num("1"));
        m.set("entries", Json::object());
    }
    return m;
}
}  // namespace

std::string store_key(const std::string& doc_id, int layer, const std::string& scheme) {
    char l[32];
    std::snprintf(l, sizeof(l), "_L%02d_", layer);
    return sha256_hex(doc_id.data(), doc_id.size()).substr(0, 16) + l + scheme;
}

void manifest_update(const std::string& dir, const std::string& doc_id, int layer,
                     const std::string& scheme, int64_t num_tokens) {
    Json m = load_manifest(dir);
    Json* entries = m.get("entries");
    if (!entries || entries->kind != Json::Obj) entries = &m.set("entries", Json::object());
    const std::string h = sha256_hex(doc_id.data(), doc_id.size());
    Json* e = entries->get(doc_id);
    if (!e || e->kind != Json::Obj) {
        Json fresh = Json::object();
        fresh.set("sha256", Json::str(h));
        fresh.set("layers", Json::object());
        e = &entries->set(doc_id, fresh);
    }
    e->set("sha256", Json::str(h));
    Json* layers = e->get("layers");
    if (!layers || layers->kind != Json::Obj) layers = &e->set("layers", Json::object());
    Json rec = Json::object();
    rec.set("key", Json::str(store_key(doc_id, layer, scheme)));
    rec.set("num_tokens", Json::num(std::to_string(num_tokens)));
    const double now = std::chrono::duration<double>(
                           std::chrono::system_clock::now().time_since_epoch()).count();
    rec.set("stored_at", Json::num(float_repr(now)));
    layers->set(std::to_string(layer) + "::" + scheme, rec);
    std::string out;
    json_dump(out, m, 0);
    write_file_atomic(manifest_path(dir), {{out.data(), out.size()}});
}

// cag_store.py:69-95: a missing entry passes; a hash or key mismatch throws.
void manifest_verify(const std::string& dir, const std::string& doc_id, int layer,
                     const std::string& scheme) {
    Json m = load_manifest(dir);
    Json* entries = m.get("entries");
    if (!entries || entries->kind != Json::Obj) return;
    Json* e = entries->get(doc_id);
    if (!e || e->kind != Json::Obj) return;
    const std::string h = sha256_hex(doc_id.data(), doc_id.size());
    Json* stored = e->get("sha256");
    if (stored && stored->kind == Json::Str && !stored->s.empty() && stored->s != h)
        throw Error("Manifest integrity error for doc_id '" + doc_id + "': stored SHA-256 " +
                    stored->s.substr(0, 8) + " != computed " + h.substr(0, 8));
    Json* layers = e->get("layers");
    if (!layers || layers->kind != Json::Obj) return;
    Json* le = layers->get(std::to_string(layer) + "::" + scheme);
    if (!le || le->kind != Json::Obj || le->obj.empty()) return;
    const std::string want = store_key(doc_id, layer, scheme);
    Json* k = le->get("key");
    const std::string got = k && k->kind == Json::Str ? k->s : std::string("None");
    if (got != want)
        throw Error("Manifest key mismatch for doc_id '" + doc_id + "' layer=" +
                    std::to_string(layer) + " scheme=" + scheme + ": stored '" + got +
                    "' != computed '" + want + "'");
}

}  // namespace store
}  // namespace tq

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
namespace {
template <class F>
int store_call(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        tq::set_last_error(e.what());
        return -2;
    } catch (...) {
        tq::set_last_error("unknown error");
        return -2;
    }
}
}  // namespace

extern "C" int tq_store_sha256_hex(const void* data, size_t n, char* out_hex65) {
    if ((!data && n) || !out_hex65) return -1;
    return store_call([&] {
        const std::string h = tq::store::sha256_hex(data, n);
        std::memcpy(out_hex65, h.c_str(), 65);
    });
}

extern "C" int tq_store_key(const char* doc_id, int layer, const char* scheme, char* out, size_t cap) {
    if (!doc_id || !scheme || !out) return -1;
    return store_call([&] {
        const std::string k = tq::store::store_key(doc_id, layer, scheme);
        if (k.size() + 1 > cap) throw tq::Error("tq_store_key: buffer too small");
        std::memcpy(out, k.c_str(), k.size() + 1);
    });
}

extern "C" int tq_store_crc32c(const void* data, size_t n, uint32_t* out) {
    if ((!data && n) || !out) return -1;
    *out = tq::store::crc32c(data, n);
    return 0;
}

extern "C" int tq_store_write_meta(const char* path, int64_t num_tokens, const int32_t* slots,
                                   int64_t num_slots, const TQStoreFormat* fmt) {
    if (!path || (!slots && num_slots) || num_slots < 0) return -1;
    return store_call([&] { tq::store::write_meta(path, num_tokens, slots, num_slots, fmt); });
}

extern "C" int tq_store_read_meta(const char* path, int64_t* num_tokens, int32_t* slots,
                                  int64_t cap, int64_t* num_slots, TQStoreFormat* fmt,
                                  int* has_fmt) {
    if (!path || !num_tokens || !num_slots || (!slots && cap > 0)) return -1;
    return store_call([&] {
        std::vector<int32_t> s;
        TQStoreFormat f;
        const bool got = tq::store::read_meta(path, num_tokens, &s, &f);
        *num_slots = (int64_t)s.size();
        if (slots && cap > 0) std::memcpy(slots, s.data(), std::min<int64_t>(cap, s.size()) * 4);
        if (has_fmt) *has_fmt = got;
        if (fmt && got) *fmt = f;
    });
}

extern "C" int tq_store_write_pool(const char* path, const uint8_t* pool, size_t pool_bytes,
                                   const TQStoreFormat* fmt) {
    if (!path || (!pool && pool_bytes) || !fmt) return -1;
    return store_call([&] { tq::store::write_pool(path, pool, pool_bytes, *fmt); });
}

extern "C" int tq_store_pool_info(const char* path, size_t* file_bytes, TQStoreFormat* fmt,
                                  int* has_footer) {
    if (!path || !file_bytes) return -1;
    return store_call([&] {
        TQStoreFormat f;
        std::memset(&f, 0, sizeof(f));
        const bool got = tq::store::pool_info(path, file_bytes, &f, nullptr);
        if (has_footer) *has_footer = got;
        if (fmt && got) *fmt = f;
    });
}

extern "C" int tq_store_read_pools(const char* const* paths, uint8_t* const* host_dst,
                                   size_t pool_bytes, int n, int threads, int verify) {
    if (n < 0 || (n > 0 && (!paths || !host_dst))) return -1;
    for (int k = 0; k < n; ++k)
        if (!paths[k] || (!host_dst[k] && pool_bytes)) return -1;
    return store_call([&] { tq::store::read_pools(paths, host_dst, pool_bytes, n, threads, verify != 0); });
}

extern "C" int tq_store_write_fp16(const char* path, int64_t num_tokens, const uint16_t* kv,
                                   int64_t numel, const int64_t* shape, int ndim) {
    if (!path || (!kv && numel) || numel < 0 || ndim < 0 || (!shape && ndim)) return -1;
    return store_call([&] {
        tq::store::write_fp16(path, num_tokens, kv, numel, std::vector<int64_t>(shape, shape + ndim));
    });
}

extern "C" int tq_store_read_fp16(const char* path, int64_t* num_tokens, uint16_t* kv, int64_t cap,
                                  int64_t* numel, int64_t* shape, int shape_cap, int* ndim) {
    if (!path || !num_tokens || !numel || (!kv && cap > 0) || (!shape && shape_cap > 0)) return -1;
    return store_call([&] {
        std::vector<uint16_t> v;
        std::vector<int64_t> sh;
        tq::store::read_fp16(path, num_tokens, &v, &sh);
        *numel = (int64_t)v.size();
        if (kv && cap > 0) std::memcpy(kv, v.data(), std::min<int64_t>(cap, v.size()) * 2);
        if (ndim) *ndim = (int)sh.size();
        if (shape)
            for (int k = 0; k < std::min<int>(shape_cap, (int)sh.size()); ++k) shape[k] = sh[k];
    });
}

extern "C" int tq_store_manifest_update(const char* store_dir, const char* doc_id, int layer,
                                        const char* scheme, int64_t num_tokens) {
    if (!store_dir || !doc_id || !scheme) return -1;
    return store_call([&] { tq::store::manifest_update(store_dir, doc_id, layer, scheme, num_tokens); });
}

extern "C" int tq_store_manifest_verify(const char* store_dir, const char* doc_id, int layer,
                                        const char* scheme) {
    if (!store_dir || !doc_id || !scheme) return -1;
    return store_call([&] { tq::store::manifest_verify(store_dir, doc_id, layer, scheme); });
}
