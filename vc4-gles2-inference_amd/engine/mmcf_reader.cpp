#include "mmcf_reader.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

namespace vgxe {

uint32_t crc32(const uint8_t* p, size_t n) {
    static uint32_t table[256];
    static bool init = false;
    if (!init) {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t c = i;
            for (int k = 0; k < 8; ++k) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
            table[i] = c;
        }
        init = true;
    }
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < n; ++i) c = table[(c ^ p[i]) & 0xFFu] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

template <typename T>
static T rd(const uint8_t* p) {
    T v;
    std::memcpy(&v, p, sizeof(T));
    return v;
}

Container::~Container() {
    if (map_) munmap(map_, size_);
    if (fd_ >= 0) close(fd_);
}

bool Container::open(const std::string& path, std::string& err) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) { err = "cannot open " + path; return false; }
    struct stat st;
    if (fstat(fd_, &st) != 0 || st.st_size < 64) { err = path + ": too short for an MMCF header"; return false; }
    size_ = (size_t)st.st_size;
    map_ = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (map_ == MAP_FAILED) { map_ = nullptr; err = "mmap failed"; return false; }
    base_ = static_cast<const uint8_t*>(map_);
    return parse(err);
}

bool Container::open_bytes(const uint8_t* data, size_t size, std::string& err) {
    base_ = data;
    size_ = size;
    return parse(err);
}

const Record* Container::find(int kind, int layer, int part) const {
    const uint16_t id = (uint16_t)(kind | (layer << 8) | (part << 14));
    auto it = recs_.find(id);
    return it == recs_.end() ? nullptr : &it->second;
}

// Header and table layout: docs/checkpoint-container.md "Header" and
// "Tensor record"; metadata keys 1, 2, 3, 11, 14, 15.
bool Container::parse(std::string& err) {
    if (size_ < 64 || std::memcmp(base_, "MMCF", 4) != 0) { err = "not an MMCF container"; return false; }
    const uint16_t version = rd<uint16_t>(base_ + 4), hsz = rd<uint16_t>(base_ + 6);
    const uint32_t n = rd<uint32_t>(base_ + 8);
    const uint32_t moff = rd<uint32_t>(base_ + 16), msize = rd<uint32_t>(base_ + 20);
    const uint64_t doff = rd<uint64_t>(base_ + 24), fsize = rd<uint64_t>(base_ + 32);
    const uint32_t hcrc = rd<uint32_t>(base_ + 40);
    if (version != 2 || hsz != 64) { err = "unsupported MMCF version " + std::to_string(version); return false; }
    if (hcrc != 0 && hcrc != crc32(base_, 40)) { err = "header crc mismatch"; return false; }
    if (fsize != size_) { err = "file size field does not match the file (truncated?)"; return false; }
    if ((uint64_t)moff + msize > size_ || doff > size_ || doff < (uint64_t)n * 48) { err = "corrupt header offsets"; return false; }
    bool have_model = false;
    for (uint64_t p = moff; p + 8 <= (uint64_t)moff + msize;) {
        const uint16_t key = rd<uint16_t>(base_ + p);
        const uint32_t len = rd<uint32_t>(base_ + p + 4);
        const uint8_t* v = base_ + p + 8;
        if (p + 8 + len > (uint64_t)moff + msize) { err = "metadata record overruns its block"; return false; }
        if (key == 1 && len >= 28) {
            meta_.dim = rd<int32_t>(v); meta_.hidden = rd<int32_t>(v + 4); meta_.layers = rd<int32_t>(v + 8);
            meta_.heads = rd<int32_t>(v + 12); meta_.kv_heads = rd<int32_t>(v + 16);
            meta_.vocab = rd<int32_t>(v + 20); meta_.seq = rd<int32_t>(v + 24);
            have_model = true;
        } else if (key == 2 && len >= 6) {
            meta_.theta = rd<float>(v); meta_.rope_half = v[4] != 0; meta_.qk_norm = v[5] != 0;
        } else if (key == 3 && len >= 4) {
            meta_.scheme = v[0]; meta_.group = v[1]; meta_.split = v[3] != 0;
        } else if (key == 11 && len >= 4) {
            meta_.rms_eps = rd<float>(v); meta_.rms_eps_stated = true;
        } else if (key == 14) {
            meta_.layer_conv.assign(v, v + len);
        } else if (key == 15) {
            meta_.hid_scale.assign(v, v + len);
        }
        p += 8 + len;
    }
    if (!have_model) { err = "metadata key 1 (model shape) missing"; return false; }
    if (meta_.layers <= 0 || meta_.layers > 63 || meta_.dim <= 0 || meta_.heads <= 0 || meta_.kv_heads <= 0 ||
        meta_.dim % meta_.heads || meta_.heads % meta_.kv_heads) {
        err = "implausible model shape"; return false;
    }
    if (!meta_.hid_scale.empty() && (int)meta_.hid_scale.size() != meta_.layers) {
        err = "metadata key 15 length is not the layer count"; return false;
    }
    for (uint8_t k : meta_.hid_scale)
        if (k > 5) { err = "metadata key 15 value over 5"; return false; }
    const uint64_t table = doff - (uint64_t)n * 48;
    for (uint32_t i = 0; i < n; ++i) {
        const uint8_t* r = base_ + table + (uint64_t)i * 48;
        Record rec;
        rec.id = rd<uint16_t>(r);
        rec.dtype = r[2];
        rec.group = r[4];
        rec.rows = rd<uint32_t>(r + 6);
        rec.cols = rd<uint32_t>(r + 10);
        const uint64_t off = rd<uint64_t>(r + 14);
        rec.bytes = rd<uint64_t>(r + 22);
        const uint32_t crc = rd<uint32_t>(r + 30);
        rec.scale = rd<float>(r + 34);
        if (doff + off + rec.bytes > size_) { err = "tensor body past the end of the file"; return false; }
        rec.body = base_ + doff + off;
        if (crc32(rec.body, rec.bytes) != crc) { err = "tensor body crc mismatch"; return false; }
        recs_[rec.id] = rec;
    }
    if (!find(T_EMB) || !find(T_EMB_SCALE) || !find(T_RMS_ATT) || !find(T_RMS_FFN) || !find(T_RMS_FINAL)) {
        err = "missing required tensors"; return false;
    }
    return true;
}

}  // namespace vgxe
