// lgx_gguf.h -- GGUF reader of Q8_0 Qwen2 checkpoints (see lgx_gguf.cpp).
#pragma once
#include <stdint.h>
#include <stdio.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/lgx.h"

namespace lgxf {

enum : uint32_t { GGML_F32 = 0, GGML_F16 = 1, GGML_Q8_0 = 8 };

struct Meta {
    uint32_t type = 0;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
};

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;   // dims[0] = row length
    uint32_t type = 0;
    uint64_t offset = 0;
};

struct Gguf {
    std::string path;
    FILE* f = nullptr;
    uint64_t alignment = 32, data_start = 0, file_size = 0;
    std::map<std::string, Meta> meta;
    std::map<std::string, TensorInfo> tensors;

    ~Gguf();
    lgx_status open(const char* path);
    const Meta* find(const std::string& key) const;
    const TensorInfo* tensor(const std::string& name) const;
    lgx_status config(int32_t max_batch, int32_t max_seq, lgx_qwen_config* cfg) const;
    // Q8_0 tensor [rows][cols] -> row-major quants [rows][cols] + scales [rows][cols/32]
    lgx_status read_q8(const std::string& name, int64_t rows, int64_t cols, int8_t* qs,
                       uint16_t* d) const;
    // F32 / F16 tensor [rows][cols] copied as stored
    lgx_status read_raw(const std::string& name, uint32_t type, int64_t rows, int64_t cols,
                        void* out) const;

  private:
    lgx_status check_extents() const;
    lgx_status seek(const std::string& name, uint32_t type, int64_t rows, int64_t cols) const;
};

}  // namespace lgxf
