// gguf.cpp — GgufReader: mmap, header / metadata / tensor-info parse, host dequantization.
#include "gguf.h"

#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>

#include "graph.h"
#include "runtime.h"
#include "tsn_common.h"

namespace tsn {

namespace {

constexpr uint32_t MAGIC = 0x46554747u;   // "GGUF" read as little-endian u32

// metadata value types of the GGUF format
enum : uint32_t {
    KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6, KV_BOOL = 7,
    KV_STRING = 8, KV_ARRAY = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12
};

// bounds-checked little-endian cursor over the mapping
struct Cursor {
    const uint8_t *p, *end;
    bool ok = true;
    bool take(void *dst, size_t n) {
        if (!ok || (size_t)(end - p) < n) return ok = false;
        if (dst) memcpy(dst, p, n);
        p += n;
        return true;
    }
    template <typename T>
    T get() {
        T v{};
        take(&v, sizeof v);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (uint64_t)(end - p)) { ok = false; return {}; }
        std::string s((const char *)p, (size_t)n);
        p += n;
        return s;
    }
};

size_t scalar_size(uint32_t t) {
    switch (t) {
    case KV_U8: case KV_I8: case KV_BOOL: return 1;
    case KV_U16: case KV_I16: return 2;
    case KV_U32: case KV_I32: case KV_F32: return 4;
    case KV_U64: case KV_I64: case KV_F64: return 8;
    default: return 0;
    }
}

} // namespace

float f16_bits_to_f32_ftz(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    uint32_t f;
    if (e == 0) f = sign;                                  // zero and subnormals -> signed zero
    else if (e == 31) f = sign | 0x7F800000u | (m << 13);  // inf / nan
    else f = sign | ((e + 112) << 23) | (m << 13);        // rebias 15 -> 127
    float out;
    memcpy(&out, &f, 4);
    return out;
}

GgufReader::~GgufReader() {
    if (map_) munmap(map_, len_);
    if (fd_ >= 0) close(fd_);
}

int GgufReader::open(const char *path) {
    TSN_REQUIRE(path && !map_, "gguf: null path or already open");
    fd_ = ::open(path, O_RDONLY);
    TSN_REQUIRE(fd_ >= 0, std::string("gguf: cannot open ") + path);
    struct stat st;
    TSN_REQUIRE(fstat(fd_, &st) == 0 && st.st_size > 24, std::string("gguf: not a GGUF file: ") + path);
    len_ = (size_t)st.st_size;
    void *m = mmap(nullptr, len_, PROT_READ, MAP_PRIVATE, fd_, 0);
    TSN_REQUIRE(m != MAP_FAILED, std::string("gguf: mmap failed: ") + path);
    map_ = m;
    return parse();
}

int GgufReader::read_at(const uint8_t *p, void *dst, size_t n) const {
    const uint8_t *base = (const uint8_t *)map_;
    TSN_REQUIRE(map_ && fd_ >= 0 && p >= base && (size_t)(p - base) <= len_ && n <= len_ - (size_t)(p - base),
                "gguf: read outside the file");
    size_t done = 0;
    while (done < n) {
        const ssize_t r = pread(fd_, (char *)dst + done, n - done, (off_t)(p - base) + (off_t)done);
        TSN_REQUIRE(r > 0, "gguf: read failed");
        done += (size_t)r;
    }
    return TSN_OK;
}

int GgufReader::parse() {
    Cursor c{(const uint8_t *)map_, (const uint8_t *)map_ + len_};
    TSN_REQUIRE(c.get<uint32_t>() == MAGIC, "gguf: bad magic");
    version_ = c.get<uint32_t>();
    TSN_REQUIRE(version_ == 2 || version_ == 3, "gguf: only versions 2 and 3 are read");
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    TSN_REQUIRE(c.ok && n_tensors < (1u << 24) && n_kv < (1u << 24), "gguf: truncated header");
    for (uint64_t i = 0; i < n_kv; ++i) {
        const std::string key = c.str();
        Kv v;
        v.type = c.get<uint32_t>();
        switch (v.type) {
        case KV_U8: v.i = c.get<uint8_t>(); break;
        case KV_I8: v.i = c.get<int8_t>(); break;
        case KV_BOOL: v.i = c.get<uint8_t>() != 0; break;
        case KV_U16: v.i = c.get<uint16_t>(); break;
        case KV_I16: v.i = c.get<int16_t>(); break;
        case KV_U32: v.i = c.get<uint32_t>(); break;
        case KV_I32: v.i = c.get<int32_t>(); break;
        case KV_U64: v.i = (int64_t)c.get<uint64_t>(); break;
        case KV_I64: v.i = c.get<int64_t>(); break;
        case KV_F32: v.f = c.get<float>(); break;
        case KV_F64: v.f = c.get<double>(); break;
        case KV_STRING: v.s = c.str(); break;
        case KV_ARRAY: {   // tokenizer vocabularies, merges and scores
            const uint32_t et = c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            v.elem = et;
            if (et == KV_STRING) {
                TSN_REQUIRE(n <= (uint64_t)(c.end - c.p) / 8, "gguf: bad string array in metadata " + key);
                v.sa.reserve((size_t)n);
                for (uint64_t k = 0; k < n && c.ok; ++k) v.sa.push_back(c.str());
            } else {
                const size_t es = scalar_size(et);
                TSN_REQUIRE(es > 0 && n <= (uint64_t)(c.end - c.p) / es, "gguf: bad array in metadata " + key);
                v.na.reserve((size_t)n);
                for (uint64_t k = 0; k < n && c.ok; ++k) {
                    switch (et) {
                    case KV_U8: v.na.push_back(c.get<uint8_t>()); break;
                    case KV_I8: v.na.push_back(c.get<int8_t>()); break;
                    case KV_BOOL: v.na.push_back(c.get<uint8_t>() != 0); break;
                    case KV_U16: v.na.push_back(c.get<uint16_t>()); break;
                    case KV_I16: v.na.push_back(c.get<int16_t>()); break;
                    case KV_U32: v.na.push_back(c.get<uint32_t>()); break;
                    case KV_I32: v.na.push_back(c.get<int32_t>()); break;
                    case KV_F32: v.na.push_back(c.get<float>()); break;
                    case KV_U64: v.na.push_back((double)c.get<uint64_t>()); break;
                    case KV_I64: v.na.push_back((double)c.get<int64_t>()); break;
                    default: v.na.push_back(c.get<double>()); break;
                    }
                }
            }
            break;
        }
        default: TSN_REQUIRE(false, "gguf: unknown metadata type for " + key);
        }
        TSN_REQUIRE(c.ok, "gguf: truncated metadata at " + key);
        kv_[key] = v;
    }
    const uint64_t align = has("general.alignment") ? (uint64_t)get_i64("general.alignment", 32) : 32;
    TSN_REQUIRE(align > 0 && (align & (align - 1)) == 0, "gguf: alignment must be a power of two");
    for (uint64_t i = 0; i < n_tensors; ++i) {
        GgufTensorInfo t;
        t.name = c.str();
        t.n_dims = c.get<uint32_t>();
        TSN_REQUIRE(c.ok && t.n_dims >= 1 && t.n_dims <= 4, "gguf: bad tensor info " + t.name);
        for (uint32_t d = 0; d < t.n_dims; ++d) t.ne[d] = c.get<uint64_t>();
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        TSN_REQUIRE(c.ok, "gguf: truncated tensor info " + t.name);
        const uint64_t n = t.numel();
        switch (t.type) {
        case GGUF_T_F32: t.nbytes = n * 4; break;
        case GGUF_T_F16: case GGUF_T_BF16: t.nbytes = n * 2; break;
        case GGUF_T_Q8_0:
            TSN_REQUIRE(t.ne[0] % 32 == 0, "gguf: Q8_0 rows must be whole 32-element blocks: " + t.name);
            t.nbytes = n / 32 * 34;
            break;
        default: t.nbytes = 0; break;   // unsupported: rejected when read
        }
        index_[t.name] = list_.size();
        list_.push_back(t);
    }
    const uint64_t hdr = (uint64_t)(c.p - (const uint8_t *)map_);
    const uint64_t data = (hdr + align - 1) & ~(align - 1);
    for (auto &t : list_) {
        TSN_REQUIRE(data + t.offset + t.nbytes <= len_ && data + t.offset >= data, "gguf: tensor past end of file: " + t.name);
        t.data = (const uint8_t *)map_ + data + t.offset;
    }
    return TSN_OK;
}

int64_t GgufReader::get_i64(const std::string &key, int64_t def) const {
    const auto it = kv_.find(key);
    if (it == kv_.end()) return def;
    return it->second.type == KV_F32 || it->second.type == KV_F64 ? (int64_t)it->second.f : it->second.i;
}

double GgufReader::get_f64(const std::string &key, double def) const {
    const auto it = kv_.find(key);
    if (it == kv_.end()) return def;
    return it->second.type == KV_F32 || it->second.type == KV_F64 ? it->second.f : (double)it->second.i;
}

std::string GgufReader::get_str(const std::string &key, const std::string &def) const {
    const auto it = kv_.find(key);
    return it == kv_.end() || it->second.type != KV_STRING ? def : it->second.s;
}

const std::vector<std::string> &GgufReader::get_arr_str(const std::string &key) const {
    static const std::vector<std::string> empty;
    const auto it = kv_.find(key);
    return it == kv_.end() || it->second.type != KV_ARRAY || it->second.elem != KV_STRING ? empty : it->second.sa;
}

std::vector<double> GgufReader::get_arr_num(const std::string &key) const {
    const auto it = kv_.find(key);
    if (it == kv_.end() || it->second.type != KV_ARRAY || it->second.elem == KV_STRING) return {};
    return it->second.na;
}

const GgufTensorInfo *GgufReader::find(const std::string &name) const {
    const auto it = index_.find(name);
    return it == index_.end() ? nullptr : &list_[it->second];
}

int GgufReader::to_f32(const GgufTensorInfo &t, float *out) const {
    TSN_REQUIRE(out && t.data, "gguf: null output or tensor");
    const uint64_t n = t.numel();
    switch (t.type) {
    case GGUF_T_F32: memcpy(out, t.data, n * 4); break;
    case GGUF_T_BF16:
        for (uint64_t i = 0; i < n; ++i) {
            uint16_t h;
            memcpy(&h, t.data + 2 * i, 2);
            const uint32_t f = (uint32_t)h << 16;
            memcpy(out + i, &f, 4);
        }
        break;
    case GGUF_T_F16:
        for (uint64_t i = 0; i < n; ++i) {
            uint16_t h;
            memcpy(&h, t.data + 2 * i, 2);
            out[i] = f16_bits_to_f32_ftz(h);
        }
        break;
    case GGUF_T_Q8_0:
        for (uint64_t b = 0; b < n / 32; ++b) {
            const uint8_t *blk = t.data + b * 34;
            uint16_t sh;
            memcpy(&sh, blk, 2);
            const float scale = f16_bits_to_f32_ftz(sh);
            for (int k = 0; k < 32; ++k) out[b * 32 + k] = scale * (float)(int8_t)blk[2 + k];
        }
        break;
    default: TSN_REQUIRE(false, "gguf: unsupported tensor type " + std::to_string(t.type) + " for " + t.name);
    }
    return TSN_OK;
}

int gguf_read_manifest(const GgufReader &g, const std::vector<ManifestEntry> &man, std::vector<float> &out) {
    TSN_REQUIRE(!man.empty(), "gguf: empty manifest");
    out.assign((size_t)(man.back().offset + man.back().numel), 0.0f);
    for (const auto &e : man) {
        const GgufTensorInfo *t = g.find(e.name);
        TSN_REQUIRE(t, "gguf: missing tensor " + e.name);
        TSN_REQUIRE((int64_t)t->numel() == e.numel, "gguf: " + e.name + " has " + std::to_string(t->numel()) +
                                                        " elements, the graph needs " + std::to_string(e.numel));
        TSN_TRY(g.to_f32(*t, out.data() + e.offset));
    }
    return TSN_OK;
}

namespace {
int wp_type_of(uint32_t t) {
    switch (t) {
    case GGUF_T_BF16: return WP_SRC_BF16;
    case GGUF_T_F32: return WP_SRC_F32;
    case GGUF_T_F16: return WP_SRC_F16;
    case GGUF_T_Q8_0: return WP_SRC_Q8_0;
    default: return -1;
    }
}

// pinned double buffer for host -> device transfers of file bytes
struct PinnedPair {
    void *buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    ~PinnedPair() {
        for (int i = 0; i < 2; ++i) {
            if (ev[i]) { hipEventSynchronize(ev[i]); hipEventDestroy(ev[i]); }
            if (buf[i]) hipHostFree(buf[i]);
        }
    }
};
constexpr size_t PIN_CHUNK = (size_t)32 << 20;
} // namespace

int gguf_stage_manifest(const GgufReader &g, const std::vector<ManifestEntry> &man, Device &dev,
                        const std::function<int(size_t, void **)> &alloc, std::map<std::string, GgufDeviceTensor> &out,
                        size_t *bytes_moved) {
    TSN_REQUIRE(!man.empty(), "gguf: empty manifest");
    struct Need {
        const GgufTensorInfo *t;
        const std::string *name;
    };
    std::vector<Need> need;
    need.reserve(man.size());
    for (const auto &e : man) {
        const GgufTensorInfo *t = g.find(e.name);
        TSN_REQUIRE(t, "gguf: missing tensor " + e.name);
        TSN_REQUIRE((int64_t)t->numel() == e.numel, "gguf: " + e.name + " has " + std::to_string(t->numel()) +
                                                        " elements, the graph needs " + std::to_string(e.numel));
        TSN_REQUIRE(wp_type_of(t->type) >= 0, "gguf: unsupported tensor type " + std::to_string(t->type) + " for " + e.name);
        TSN_REQUIRE(t->type != GGUF_T_Q8_0 || t->numel() % 32 == 0, "gguf: Q8_0 tensor " + e.name + " is not whole blocks");
        need.push_back(Need{t, &e.name});
    }
    // runs of tensors adjacent in the file (gaps of at most 4 KiB, the alignment padding, travel along)
    std::sort(need.begin(), need.end(), [](const Need &a, const Need &b) { return a.t->data < b.t->data; });
    struct Run {
        const uint8_t *src;
        size_t bytes, dst;
    };
    std::vector<Run> runs;
    std::vector<size_t> run_of(need.size());
    size_t total = 0;
    for (size_t i = 0; i < need.size(); ++i) {
        const uint8_t *a = need[i].t->data, *b = a + need[i].t->nbytes;
        if (!runs.empty() && a >= runs.back().src && a <= runs.back().src + runs.back().bytes + 4096) {
            Run &r = runs.back();
            const size_t end = std::max(r.bytes, (size_t)(b - r.src));
            total += end - r.bytes;
            r.bytes = end;
        } else {
            total = (total + 255) & ~(size_t)255;   // each run starts 256-byte aligned on the device
            runs.push_back(Run{a, (size_t)(b - a), total});
            total += runs.back().bytes;
        }
        run_of[i] = runs.size() - 1;
    }
    void *stage = nullptr;
    TSN_TRY(alloc(total, &stage));
    TSN_TRY(dev.make_current());
    const hipStream_t st = dev.stream();
    PinnedPair pin;
    for (int i = 0; i < 2; ++i) {
        TSN_HIP_CHECK(hipHostMalloc(&pin.buf[i], PIN_CHUNK, hipHostMallocDefault));
        TSN_HIP_CHECK(hipEventCreateWithFlags(&pin.ev[i], hipEventDisableTiming));
    }
    int slot = 0;
    for (const Run &r : runs)
        for (size_t off = 0; off < r.bytes; off += PIN_CHUNK) {
            const size_t n = std::min(PIN_CHUNK, r.bytes - off);
            if (pin.used[slot]) TSN_HIP_CHECK(hipEventSynchronize(pin.ev[slot]));   // its previous DMA is done
            TSN_TRY(g.read_at(r.src + off, pin.buf[slot], n));
            TSN_HIP_CHECK(hipMemcpyAsync((char *)stage + r.dst + off, pin.buf[slot], n, hipMemcpyHostToDevice, st));
            TSN_HIP_CHECK(hipEventRecord(pin.ev[slot], st));
            pin.used[slot] = true;
            slot ^= 1;
        }
    TSN_HIP_CHECK(hipStreamSynchronize(st));
    out.clear();
    for (size_t i = 0; i < need.size(); ++i) {
        const Run &r = runs[run_of[i]];
        const char *p = (const char *)stage + r.dst + (need[i].t->data - r.src);
        out[*need[i].name] = GgufDeviceTensor{p, wp_type_of(need[i].t->type)};
    }
    if (bytes_moved) *bytes_moved = total;
    return TSN_OK;
}

} // namespace tsn
