// MMCF v2 container reader for the engine: maps the file, validates the
// header, metadata and tensor table (CRCs, sizes), and hands out the tensor
// bodies in place.  Semantics follow Model::load / read_tables
// (engine/src/model.cpp:873-1304) and docs/checkpoint-container.md:62-271.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace vgxe {

enum Dtype { DT_F32 = 0, DT_I16 = 1, DT_Q8U8 = 2, DT_Q8I8 = 3, DT_Q4 = 4, DT_BLOB = 5, DT_Q6 = 6, DT_T3 = 7 };
enum Kind {
    T_EMB = 1, T_EMB_SCALE = 2, T_RMS_ATT = 3, T_RMS_FFN = 4, T_RMS_FINAL = 5, T_Q_NORM = 6, T_K_NORM = 7,
    T_QKV = 0x10, T_WO = 0x11, T_W1 = 0x12, T_W3 = 0x13, T_W13 = 0x14, T_W2 = 0x15,
    T_CONV_IN = 0x17, T_CONV_W = 0x18, T_CONV_OUT = 0x19, T_LOGITS = 0x20
};

struct Record {
    uint16_t id = 0;
    uint8_t dtype = 0, group = 0;
    uint32_t rows = 0, cols = 0;
    float scale = 0.0f;
    const uint8_t* body = nullptr;
    uint64_t bytes = 0;
};

struct ModelMeta {
    int dim = 0, hidden = 0, layers = 0, heads = 0, kv_heads = 0, vocab = 0, seq = 0;
    float theta = 10000.0f;
    bool rope_half = false, qk_norm = false;
    int scheme = 1;      // 0 i16, 1 q8, 2 q4, 3 t3
    int group = 0;
    bool split = false;  // separate w1/w3 records
    float rms_eps = 1e-5f;
    bool rms_eps_stated = false;
    std::vector<uint8_t> layer_conv;  // key 14
    std::vector<uint8_t> hid_scale;   // key 15
    int head_dim() const { return heads ? dim / heads : 0; }
    int kv_dim() const { return kv_heads * head_dim(); }
};

class Container {
public:
    ~Container();
    // Returns false with `err` set on any refusal (bad magic, version, CRC,
    // truncation, missing tensors).
    bool open(const std::string& path, std::string& err);
    bool open_bytes(const uint8_t* data, size_t size, std::string& err);
    const ModelMeta& meta() const { return meta_; }
    const Record* find(int kind, int layer = 0, int part = 0) const;
    size_t file_size() const { return size_; }

private:
    bool parse(std::string& err);
    const uint8_t* base_ = nullptr;
    size_t size_ = 0;
    void* map_ = nullptr;
    int fd_ = -1;
    ModelMeta meta_;
    std::map<uint16_t, Record> recs_;
};

uint32_t crc32(const uint8_t* p, size_t n);

}  // namespace vgxe
