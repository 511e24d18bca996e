// Memory-mapped safetensors reader (header parse + zero-copy tensor bytes).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/brain_hip.h"

namespace bh {

int fail(int code, const char* fmt, ...);

enum StDtype { ST_OTHER = 0, ST_F32 = 1, ST_U32 = 2, ST_I8 = 3, ST_U8 = 4, ST_F16 = 5, ST_BF16 = 6, ST_I32 = 7 };
size_t st_dtype_size(int dtype);

struct StTensor {
    std::string name;
    int dtype = ST_OTHER;
    std::vector<uint64_t> shape;
    uint64_t begin = 0, end = 0;  // byte range within the data section
};

class StFile {
   public:
    StFile() = default;
    StFile(const StFile&) = delete;
    StFile& operator=(const StFile&) = delete;
    ~StFile();
    bool open(const std::string& path, std::string* err);
    const StTensor* find(const std::string& name) const;
    const uint8_t* bytes(const StTensor& t) const;
    const std::map<std::string, StTensor>& tensors() const { return tensors_; }

   private:
    void* map_ = nullptr;
    size_t size_ = 0;
    const uint8_t* data_ = nullptr;
    std::map<std::string, StTensor> tensors_;
};

}  // namespace bh
