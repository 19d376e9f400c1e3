// gguf.h — read-only GGUF checkpoint reader (host C++, mmap).
//
// Replaces tn::GgufFile / tn::to_f32 (src/gguf.h:42-86, src/gguf.cpp): GGUF v2/v3 header, typed
// key-value metadata, tensor infos (ne[0] fastest), data section at the file's alignment
// (general.alignment, default 32). Tensor payloads are read in place from the mapping, either
// copied raw to device memory (gguf_stage_manifest; the device converts them) or dequantized on the
// host to f32 with the reference's semantics: F32 as is, BF16 exact, F16 and the Q8_0 block scale
// with subnormals flushed to zero, Q8_0 = scale * int8.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <functional>
#include <map>
#include <string>
#include <vector>

namespace tsn {

enum GgufTensorType : uint32_t { GGUF_T_F32 = 0, GGUF_T_F16 = 1, GGUF_T_Q8_0 = 8, GGUF_T_BF16 = 30 };

struct GgufTensorInfo {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1};   // ne[0] fastest
    uint32_t type = GGUF_T_F32;
    uint64_t offset = 0;             // from the start of the data section
    uint64_t nbytes = 0;
    const uint8_t *data = nullptr;
    uint64_t numel() const { return ne[0] * ne[1] * ne[2] * ne[3]; }
};

class GgufReader {
public:
    ~GgufReader();
    // map and parse; TSN_* status, message in last_error
    int open(const char *path);
    bool has(const std::string &key) const { return kv_.count(key) != 0; }
    int64_t get_i64(const std::string &key, int64_t def) const;
    double get_f64(const std::string &key, double def) const;
    std::string get_str(const std::string &key, const std::string &def) const;
    // array metadata (empty when absent or of another element type): strings, and any numeric
    // element type widened to double
    const std::vector<std::string> &get_arr_str(const std::string &key) const;
    std::vector<double> get_arr_num(const std::string &key) const;
    const GgufTensorInfo *find(const std::string &name) const;
    const std::vector<GgufTensorInfo> &tensors() const { return list_; }
    uint32_t version() const { return version_; }
    // dequantize to f32 (out holds numel floats)
    int to_f32(const GgufTensorInfo &t, float *out) const;
    // n bytes of the file starting at p (an address inside the mapping), read with pread into dst:
    // the bytes go from the page cache straight to dst, without faulting the mapping in
    int read_at(const uint8_t *p, void *dst, size_t n) const;

private:
    struct Kv {
        uint32_t type = 0;
        int64_t i = 0;
        double f = 0;
        std::string s;
        uint32_t elem = 0;                // array element type
        std::vector<std::string> sa;      // string array
        std::vector<double> na;           // numeric array
    };
    int fd_ = -1;
    void *map_ = nullptr;
    size_t len_ = 0;
    uint32_t version_ = 0;
    std::map<std::string, Kv> kv_;
    std::vector<GgufTensorInfo> list_;
    std::map<std::string, size_t> index_;
    int parse();
};

// f16 bits -> f32 with subnormals flushed to signed zero (the reference's host conversion)
float f16_bits_to_f32_ftz(uint16_t h);

struct ManifestEntry;
// every tensor of a manifest looked up by name in the file, its element count checked, dequantized
// to f32 into out at the manifest offsets (WeightSet::load's name map, src/net.mm:126-140)
int gguf_read_manifest(const GgufReader &g, const std::vector<ManifestEntry> &man, std::vector<float> &out);

// One manifest tensor's raw GGUF payload in device memory: its address and its encoding as a
// weight_prep source type (WP_SRC_BF16 / F32 / F16 / Q8_0).
struct GgufDeviceTensor {
    const void *p;
    int type;
};
class Device;
// The raw payloads of every tensor of a manifest, copied as stored in the file (no host
// conversion) from the mapping to one device buffer that `alloc` provides: tensors are looked up
// by name, their element counts and types checked, and each run of tensors that lie next to each
// other in the file goes over as one transfer, read from the file into two pinned host buffers in
// turn, so the read of one chunk overlaps the previous chunk's DMA. The device buffer holds only the needed runs;
// out maps each name to its bytes there. Bytes moved over PCIe are returned in *bytes_moved.
int gguf_stage_manifest(const GgufReader &g, const std::vector<ManifestEntry> &man, Device &dev,
                        const std::function<int(size_t, void **)> &alloc, std::map<std::string, GgufDeviceTensor> &out,
                        size_t *bytes_moved);

} // namespace tsn
