// mcf.cpp -- MCF reader/writer, deterministic weight generator and the k4
// producer (host code of libmantle_hip.so).
#include "mcf.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <thread>

namespace mantle {

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }
static inline uint64_t rd64(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }

static constexpr uint64_t kHeaderSize = 40;
static constexpr uint64_t kSectionAlign = 8;  // pkg/mcf/utils.go:8 mcfAlign

int64_t k4_payload_bytes(int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0) return -1;
    int64_t bpr = (cols + 31) / 32, spr = (bpr + 7) / 8;
    int64_t sub_off = (rows * spr * 2 + 63) & ~(int64_t)63;
    int64_t data_off = (sub_off + rows * bpr + 63) & ~(int64_t)63;
    return data_off + rows * bpr * 16;
}

static uint64_t elem_size(uint16_t dt) {
    switch (dt) {
        case kDTypeF32: return 4;
        case kDTypeF16:
        case kDTypeBF16: return 2;
        case 4: return 8;           // F64
        case 5: case 6: return 1;   // I8, U8
        case 7: case 8: return 2;   // I16, U16
        case 9: case 10: return 4;  // I32, U32
        case 11: case 12: return 8; // I64, U64
        default: return 0;
    }
}

// ---------------------------------------------------------------------------
// Reader

McfFile::~McfFile() {
    if (base_ && owned_) munmap(base_, size_);
}

int McfFile::find(const std::string& name) const {
    // Index entries are sorted by name (TensorIndexFlagSortedByName).
    auto it = std::lower_bound(tensors_.begin(), tensors_.end(), name,
                               [](const McfTensor& t, const std::string& n) { return t.name < n; });
    if (it != tensors_.end() && it->name == name) return (int)(it - tensors_.begin());
    for (size_t i = 0; i < tensors_.size(); i++)
        if (tensors_[i].name == name) return (int)i;
    return -1;
}

const McfSection* McfFile::section(uint32_t type) const {
    for (auto& s : sections_)
        if (s.type == type) return &s;
    return nullptr;
}

bool McfFile::open(const std::string& path, std::string* err) {
    auto fail = [&](const char* m) {
        if (err) *err = m;
        return false;
    };
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return fail("mcf: cannot open file");
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < (off_t)kHeaderSize) {
        ::close(fd);
        return fail("mcf: file too small");
    }
    size_ = (uint64_t)st.st_size;
    void* p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) return fail("mcf: mmap failed");
    base_ = (uint8_t*)p;
    owned_ = true;
    return parse(err);
}

bool McfFile::open_image(const uint8_t* data, uint64_t size, std::string* err) {
    if (!data || size < kHeaderSize) {
        if (err) *err = "mcf: image too small";
        return false;
    }
    base_ = const_cast<uint8_t*>(data);
    size_ = size;
    owned_ = false;
    return parse(err);
}

bool McfFile::parse(std::string* err) {
    auto fail = [&](const char* m) {
        if (err) *err = m;
        return false;
    };
    // Header (pkg/mcf/header.go)
    if (memcmp(base_, "MCF\0", 4) != 0) return fail("mcf: bad magic");
    uint16_t major = rd16(base_ + 4);
    uint32_t hsize = rd32(base_ + 8), nsec = rd32(base_ + 12);
    uint64_t dir = rd64(base_ + 16), fsize = rd64(base_ + 24);
    if (major != 1) return fail("mcf: unsupported major version");
    if (hsize < kHeaderSize || nsec == 0) return fail("mcf: invalid header");
    if (fsize != size_) return fail("mcf: file size mismatch");
    if (dir > size_ || dir + (uint64_t)nsec * 24 > size_) return fail("mcf: section directory out of range");
    for (uint32_t i = 0; i < nsec; i++) {
        const uint8_t* e = base_ + dir + 24ull * i;
        McfSection s{rd32(e), rd32(e + 4), rd64(e + 8), rd64(e + 16)};
        if (s.off % kSectionAlign) return fail("mcf: section offset not aligned");
        if (s.off > size_ || s.off + s.size > size_ || s.off + s.size < s.off) return fail("mcf: section out of range");
        sections_.push_back(s);
    }
    const McfSection* idx = section(kSecTensorIndex);
    const McfSection* td = section(kSecTensorData);
    if (!idx) return fail("mcf: missing tensor index section");
    if (!td) return fail("mcf: missing tensor data section");
    // Tensor index (pkg/mcf/tensor_index.go:132-220)
    const uint8_t* s = base_ + idx->off;
    const uint64_t slen = idx->size;
    if (slen < 48) return fail("mcf: tensor index too small");
    uint32_t ver = rd32(s), count = rd32(s + 8), ndims = rd32(s + 12);
    uint64_t eoff = rd64(s + 16), doff = rd64(s + 24), stroff = rd64(s + 32), strsz = rd64(s + 40);
    if (ver != 1 || count == 0) return fail("mcf: bad tensor index header");
    if (eoff + 40ull * count > slen || doff + 8ull * ndims > slen || stroff + strsz > slen)
        return fail("mcf: tensor index tables out of range");
    tensors_.reserve(count);
    for (uint32_t i = 0; i < count; i++) {
        const uint8_t* e = s + eoff + 40ull * i;
        uint32_t noff = rd32(e), nlen = rd32(e + 4), dt = rd32(e + 8), rank = rd32(e + 12), dimoff = rd32(e + 16);
        if (dt > 0xFFFF || (uint64_t)noff + nlen > strsz || (uint64_t)dimoff + rank > ndims)
            return fail("mcf: corrupt tensor index entry");
        McfTensor t;
        t.name.assign((const char*)s + stroff + noff, nlen);
        t.dtype = (uint16_t)dt;
        for (uint32_t d = 0; d < rank; d++) t.shape.push_back(rd64(s + doff + 8ull * (dimoff + d)));
        t.off = rd64(e + 24);
        t.size = rd64(e + 32);
        if (t.off < td->off || t.off + t.size > td->off + td->size || t.off + t.size < t.off)
            return fail("mcf: tensor data out of bounds");
        uint64_t want = 0;
        if (t.dtype == kDTypeK4) {
            if (t.shape.size() != 2) return fail("mcf: quant tensors must be rank-2");
            int64_t w = k4_payload_bytes((int64_t)t.shape[0], (int64_t)t.shape[1]);
            if (w < 0) return fail("mcf: invalid quant tensor shape");
            want = (uint64_t)w;
        } else {
            uint64_t es = elem_size(t.dtype);
            if (!es) return fail("mcf: unsupported tensor dtype");
            want = es;
            for (auto d : t.shape) want *= d;
        }
        if (want != t.size) return fail("mcf: tensor data size mismatch");
        tensors_.push_back(std::move(t));
    }
    return true;
}

// ---------------------------------------------------------------------------
// Writer

bool McfWriter::put(const void* p, uint64_t n) {
    if (n && fwrite(p, 1, n, f_) != n) return false;
    pos_ += n;
    return true;
}

bool McfWriter::pad_to(uint64_t align) {
    static const uint8_t zeros[64] = {0};
    while (pos_ % align) {
        uint64_t k = std::min<uint64_t>(align - pos_ % align, sizeof zeros);
        if (!put(zeros, k)) return false;
    }
    return true;
}

bool McfWriter::open(const std::string& path, std::string* err) {
    f_ = fopen(path.c_str(), "wb");
    if (!f_) {
        if (err) *err = "mcf: cannot create file";
        return false;
    }
    uint8_t zeros[kHeaderSize] = {0};
    return put(zeros, kHeaderSize) && pad_to(kSectionAlign);
}

bool McfWriter::write_section(uint32_t type, uint32_t version, const void* data, uint64_t n) {
    if (!pad_to(kSectionAlign)) return false;
    McfSection s{type, version, pos_, n};
    if (!put(data, n)) return false;
    secs_.push_back(s);
    return true;
}

bool McfWriter::begin_tensor_data() {
    if (!pad_to(kSectionAlign)) return false;
    td_start_ = pos_;
    return true;
}

bool McfWriter::add_tensor(const std::string& name, uint16_t dtype, const std::vector<uint64_t>& shape,
                           const void* data, uint64_t n, bool quant, float min_clip, float max_clip) {
    if (!pad_to(64)) return false;  // cmd/mantle/quantize.go:288 td.Align(64)
    McfTensor t;
    t.name = name;
    t.dtype = dtype;
    t.shape = shape;
    t.off = pos_;
    t.size = n;
    if (!put(data, n)) return false;
    recs_.push_back(t);
    if (quant) qrecs_.push_back({name, min_clip, max_clip});
    return true;
}

bool McfWriter::end_tensor_data() {
    secs_.push_back({kSecTensorData, 1, td_start_, pos_ - td_start_});
    return true;
}

bool McfWriter::finalise(uint64_t flags) {
    // Tensor index (EncodeTensorIndexSection, pkg/mcf/tensor_index.go:368-470): sorted by name.
    std::sort(recs_.begin(), recs_.end(), [](const McfTensor& a, const McfTensor& b) { return a.name < b.name; });
    std::vector<uint64_t> dims;
    std::string strings;
    std::vector<uint8_t> entries(40 * recs_.size(), 0);
    for (size_t i = 0; i < recs_.size(); i++) {
        const McfTensor& r = recs_[i];
        uint8_t* e = entries.data() + 40 * i;
        uint32_t noff = (uint32_t)strings.size(), nlen = (uint32_t)r.name.size();
        uint32_t dt = r.dtype, rank = (uint32_t)r.shape.size(), dimoff = (uint32_t)dims.size();
        memcpy(e, &noff, 4);
        memcpy(e + 4, &nlen, 4);
        memcpy(e + 8, &dt, 4);
        memcpy(e + 12, &rank, 4);
        memcpy(e + 16, &dimoff, 4);
        memcpy(e + 24, &r.off, 8);
        memcpy(e + 32, &r.size, 8);
        strings += r.name;
        dims.insert(dims.end(), r.shape.begin(), r.shape.end());
    }
    std::vector<uint8_t> idx(48);
    uint32_t h32[4] = {1u, 3u /* sorted | utf8 */, (uint32_t)recs_.size(), (uint32_t)dims.size()};
    uint64_t eoff = 48, doff = eoff + entries.size(), stroff = doff + 8 * dims.size(), strsz = strings.size();
    memcpy(idx.data(), h32, 16);
    memcpy(idx.data() + 16, &eoff, 8);
    memcpy(idx.data() + 24, &doff, 8);
    memcpy(idx.data() + 32, &stroff, 8);
    memcpy(idx.data() + 40, &strsz, 8);
    idx.insert(idx.end(), entries.begin(), entries.end());
    const uint8_t* dp = reinterpret_cast<const uint8_t*>(dims.data());
    idx.insert(idx.end(), dp, dp + 8 * dims.size());
    idx.insert(idx.end(), strings.begin(), strings.end());
    if (!write_section(kSecTensorIndex, 1, idx.data(), idx.size())) return false;
    // QuantInfo (pkg/mcf/quantinfo.go): 8-byte header + 24-byte records, TensorIndex = sorted position.
    if (!qrecs_.empty()) {
        std::vector<uint8_t> q(8 + 24 * qrecs_.size(), 0);
        uint32_t qh[2] = {1u, (uint32_t)qrecs_.size()};
        memcpy(q.data(), qh, 8);
        size_t k = 0;
        for (size_t i = 0; i < recs_.size(); i++) {
            for (auto& qr : qrecs_) {
                if (qr.name != recs_[i].name) continue;
                uint8_t* e = q.data() + 8 + 24 * k++;
                uint32_t ti = (uint32_t)i;
                uint16_t bs = 32, ss = 256;
                memcpy(e, &ti, 4);
                e[4] = (uint8_t)kDTypeK4;
                e[5] = 0;  // DomainWeights
                memcpy(e + 6, &bs, 2);
                memcpy(e + 8, &ss, 2);
                memcpy(e + 16, &qr.min_clip, 4);
                memcpy(e + 20, &qr.max_clip, 4);
            }
        }
        if (!write_section(kSecQuantInfo, 1, q.data(), q.size())) return false;
    }
    std::sort(secs_.begin(), secs_.end(), [](const McfSection& a, const McfSection& b) { return a.type < b.type; });
    if (!pad_to(kSectionAlign)) return false;
    uint64_t dir = pos_;
    for (auto& s : secs_) {
        uint8_t e[24];
        memcpy(e, &s.type, 4);
        memcpy(e + 4, &s.version, 4);
        memcpy(e + 8, &s.off, 8);
        memcpy(e + 16, &s.size, 8);
        if (!put(e, 24)) return false;
    }
    uint64_t fsize = pos_;
    uint8_t h[kHeaderSize] = {0};
    memcpy(h, "MCF\0", 4);
    uint16_t major = 1, minor = 1;
    uint32_t hsize = (uint32_t)kHeaderSize, nsec = (uint32_t)secs_.size();
    memcpy(h + 4, &major, 2);
    memcpy(h + 6, &minor, 2);
    memcpy(h + 8, &hsize, 4);
    memcpy(h + 12, &nsec, 4);
    memcpy(h + 16, &dir, 8);
    memcpy(h + 24, &fsize, 8);
    memcpy(h + 32, &flags, 8);
    bool ok = fseek(f_, 0, SEEK_SET) == 0 && fwrite(h, 1, kHeaderSize, f_) == kHeaderSize;
    ok = (fclose(f_) == 0) && ok;
    f_ = nullptr;
    return ok;
}

// ---------------------------------------------------------------------------
// Deterministic N(0, std) weights: splitmix64 counter stream + Box-Muller.

uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t fnv1a64(const std::string& s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h;
}

template <class F>
static void parallel_for(int64_t n, int threads, F f) {
    if (threads <= 1 || n < 4096) {
        f(0, n);
        return;
    }
    std::vector<std::thread> ts;
    int64_t chunk = (n + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        int64_t a = t * chunk, b = std::min(n, a + chunk);
        if (a >= b) break;
        ts.emplace_back([=] { f(a, b); });
    }
    for (auto& t : ts) t.join();
}

void fill_normal(float* dst, int64_t n, uint64_t tseed, float std_dev, int threads) {
    const int64_t pairs = (n + 1) / 2;
    parallel_for(pairs, threads, [=](int64_t a, int64_t b) {
        const double two_pi = 6.283185307179586476925286766559;
        for (int64_t k = a; k < b; k++) {
            uint64_t r1 = splitmix64(tseed + 2 * (uint64_t)k), r2 = splitmix64(tseed + 2 * (uint64_t)k + 1);
            double u1 = (double)((r1 >> 11) + 1) * (1.0 / 9007199254740992.0);
            double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);
            double rad = sqrt(-2.0 * log(u1));
            dst[2 * k] = (float)(rad * cos(two_pi * u2) * std_dev);
            if (2 * k + 1 < n) dst[2 * k + 1] = (float)(rad * sin(two_pi * u2) * std_dev);
        }
    });
}

// ---------------------------------------------------------------------------
// k4 producer: cmd/mantle/quantize.go:352-398 (quantizeTensor) + :530-651 (quantizeK, bits 4).

static inline int32_t go_round_f32(float v) { return (int32_t)roundf(v); }

int quantize_k4(const float* src, int64_t rows, int64_t cols, uint8_t* payload, float* min_clip, float* max_clip,
                int threads) {
    const int64_t psize = k4_payload_bytes(rows, cols);
    if (psize < 0) return -1;
    float mn = INFINITY, mx = -INFINITY;
    for (int64_t i = 0; i < rows * cols; i++) {
        float v = src[i];
        if (std::isnan(v) || std::isinf(v)) return -2;
        mn = v < mn ? v : mn;
        mx = v > mx ? v : mx;
    }
    const float amn = fabsf(mn), amx = fabsf(mx);
    const float maxabs = amn > amx ? amn : amx;
    const float lo = -maxabs, hi = maxabs;
    if (min_clip) *min_clip = lo;
    if (max_clip) *max_clip = hi;
    memset(payload, 0, (size_t)psize);
    const int64_t bpr = (cols + 31) / 32, spr = (bpr + 7) / 8;
    const int64_t sub_off = (rows * spr * 2 + 63) & ~(int64_t)63;
    const int64_t data_off = (sub_off + rows * bpr + 63) & ~(int64_t)63;
    uint8_t* super_p = payload;
    uint8_t* sub_p = payload + sub_off;
    uint8_t* data_p = payload + data_off;
    auto clampv = [&](float v) { return v < lo ? lo : (v > hi ? hi : v); };
    parallel_for(rows, threads, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; r++) {
            const int64_t row_base = r * cols, row_limit = row_base + cols;
            for (int64_t s = 0; s < spr; s++) {
                float bs[8];
                float max_scale = 0.0f;
                for (int b = 0; b < 8; b++) {
                    const int64_t block = s * 8 + b;
                    bs[b] = 0.0f;
                    if (block >= bpr) continue;
                    float ma = 0.0f;
                    for (int i = 0; i < 32; i++) {
                        const int64_t idx = row_base + block * 32 + i;
                        const float v = idx < row_limit ? clampv(src[idx]) : 0.0f;
                        const float av = fabsf(v);
                        if (av > ma) ma = av;
                    }
                    if (ma == 0.0f) continue;
                    bs[b] = ma / 7.0f;
                    if (bs[b] > max_scale) max_scale = bs[b];
                }
                const float super_scale = max_scale;
                // Float32ToFloat16 (internal/backend/simd/float16.go:7-46): truncating, FTZ.
                uint32_t bits;
                memcpy(&bits, &super_scale, 4);
                uint16_t h;
                {
                    uint16_t sign = (uint16_t)((bits >> 31) & 1u);
                    int exp = (int)((bits >> 23) & 0xFFu);
                    uint32_t mant = bits & 0x7FFFFFu;
                    uint16_t oe = 0, om = 0;
                    if (exp == 0) {
                        oe = 0;
                        om = 0;
                    } else if (exp == 0xFF) {
                        oe = 0x1F;
                        om = mant ? 0x200 : 0;
                    } else {
                        int ne = exp - 127 + 15;
                        if (ne >= 31) oe = 0x1F;
                        else if (ne > 0) { oe = (uint16_t)ne; om = (uint16_t)(mant >> 13); }
                    }
                    h = (uint16_t)((sign << 15) | (oe << 10) | om);
                }
                const int64_t si = r * spr + s;
                super_p[si * 2] = (uint8_t)(h & 0xFF);
                super_p[si * 2 + 1] = (uint8_t)(h >> 8);
                for (int b = 0; b < 8; b++) {
                    const int64_t block = s * 8 + b;
                    if (block >= bpr) continue;
                    const int64_t bi = r * bpr + block;
                    uint8_t u6 = 0;
                    if (bs[b] > 0 && super_scale > 0) {
                        int u = (int)go_round_f32((bs[b] / super_scale) * 32.0f);
                        u = u < 1 ? 1 : (u > 63 ? 63 : u);
                        u6 = (uint8_t)u;
                    }
                    sub_p[bi] = u6 & 0x3F;
                    float scale = 0.0f;
                    if (u6 > 0 && super_scale > 0) scale = super_scale * ((float)u6 / 32.0f);
                    const float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
                    uint8_t* dst = data_p + bi * 16;
                    for (int i = 0; i < 32; i++) {
                        const int64_t idx = row_base + block * 32 + i;
                        const float v = idx < row_limit ? clampv(src[idx]) : 0.0f;
                        int32_t q = 0;
                        if (scale != 0.0f) {
                            q = go_round_f32(v * inv);
                            q = q > 7 ? 7 : (q < -7 ? -7 : q);
                        }
                        dst[i >> 1] |= (uint8_t)(((uint8_t)(int8_t)q & 0x0F) << ((i & 1) * 4));
                    }
                }
            }
        }
    });
    return 0;
}

}  // namespace mantle
