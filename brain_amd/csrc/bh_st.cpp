// The int8 checkpoint format on disk: a safetensors file in which every
// quantized linear `name` is a U32 tensor [n, k/4] (4 int8 per word, little
// endian along K, the packed layout of crates/model/src/int8.rs:33-59) with an
// F32 sibling `name.scale` [n]; every other tensor is F32
// (crates/qwen3omnimoe/src/import.rs:420-425 plans it this way). The reader
// maps the file and parses only the JSON header; tensor bytes are read
// straight from the mapping in row-aligned chunks, so host memory stays
// bounded by the mapping (crates/model/src/int8.rs:131-187,
// crates/checkpoint/src/weightio.rs).
#include "bh_st.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cstdlib>
#include <cstring>

namespace bh {

namespace {

// Minimal JSON reader for the safetensors header: objects, arrays, strings
// (with escapes), integers. Values of other kinds in __metadata__ are skipped.
struct Json {
    const char* p;
    const char* end;
    bool ok = true;

    void ws() {
        while (p < end && isspace((unsigned char)*p)) ++p;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) {
            ++p;
            return true;
        }
        return false;
    }
    bool str(std::string* out) {
        ws();
        if (p >= end || *p != '"') return ok = false;
        ++p;
        std::string s;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                ++p;
                if (p >= end) return ok = false;
                switch (*p) {
                    case 'n': s += '\n'; break;
                    case 't': s += '\t'; break;
                    case 'r': s += '\r'; break;
                    case 'b': s += '\b'; break;
                    case 'f': s += '\f'; break;
                    case 'u':
                        // Keep \uXXXX verbatim: tensor names here are ASCII.
                        s += "\\u";
                        break;
                    default: s += *p;
                }
                ++p;
            } else {
                s += *p++;
            }
        }
        if (p >= end) return ok = false;
        ++p;
        if (out) *out = s;
        return true;
    }
    bool num(uint64_t* out) {
        ws();
        if (p >= end || !isdigit((unsigned char)*p)) return ok = false;
        uint64_t v = 0;
        while (p < end && isdigit((unsigned char)*p)) {
            const uint64_t d = (uint64_t)(*p++ - '0');
            if (v > (UINT64_MAX - d) / 10) return ok = false;
            v = v * 10 + d;
        }
        if (out) *out = v;
        return true;
    }
    bool skip() {  // any value
        ws();
        if (p >= end) return ok = false;
        if (*p == '"') return str(nullptr);
        if (*p == '{') {
            ++p;
            if (eat('}')) return true;
            do {
                if (!str(nullptr) || !eat(':') || !skip()) return ok = false;
            } while (eat(','));
            return eat('}') || (ok = false);
        }
        if (*p == '[') {
            ++p;
            if (eat(']')) return true;
            do {
                if (!skip()) return ok = false;
            } while (eat(','));
            return eat(']') || (ok = false);
        }
        while (p < end && *p != ',' && *p != '}' && *p != ']' && !isspace((unsigned char)*p)) ++p;  // number/true/false/null
        return true;
    }
};

int dtype_code(const std::string& s) {
    if (s == "F32") return ST_F32;
    if (s == "U32") return ST_U32;
    if (s == "I8") return ST_I8;
    if (s == "U8") return ST_U8;
    if (s == "F16") return ST_F16;
    if (s == "BF16") return ST_BF16;
    if (s == "I32") return ST_I32;
    return ST_OTHER;
}

}  // namespace

size_t st_dtype_size(int dtype) {
    switch (dtype) {
        case ST_F32:
        case ST_U32:
        case ST_I32: return 4;
        case ST_F16:
        case ST_BF16: return 2;
        case ST_I8:
        case ST_U8: return 1;
        default: return 0;
    }
}

StFile::~StFile() {
    if (map_ && map_ != MAP_FAILED) munmap(map_, size_);
}

bool StFile::open(const std::string& path, std::string* err) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
        *err = "cannot open " + path;
        return false;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 8) {
        ::close(fd);
        *err = path + ": not a safetensors file (too short)";
        return false;
    }
    size_ = (size_t)st.st_size;
    map_ = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map_ == MAP_FAILED) {
        map_ = nullptr;
        *err = "mmap failed for " + path;
        return false;
    }
    const uint8_t* b = static_cast<const uint8_t*>(map_);
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | b[i];
    if (hlen > size_ - 8) {
        *err = path + ": header length exceeds the file";
        return false;
    }
    data_ = b + 8 + hlen;
    const size_t data_size = size_ - 8 - hlen;
    Json j{reinterpret_cast<const char*>(b + 8), reinterpret_cast<const char*>(b + 8 + hlen)};
    if (!j.eat('{')) {
        *err = path + ": header is not a JSON object";
        return false;
    }
    if (!j.eat('}')) {
        do {
            std::string name;
            if (!j.str(&name) || !j.eat(':')) break;
            if (name == "__metadata__") {
                if (!j.skip()) break;
                continue;
            }
            StTensor t;
            t.name = name;
            if (!j.eat('{')) break;
            bool have_dtype = false, have_shape = false, have_off = false;
            do {
                std::string key;
                if (!j.str(&key) || !j.eat(':')) break;
                if (key == "dtype") {
                    std::string d;
                    if (!j.str(&d)) break;
                    t.dtype = dtype_code(d);
                    have_dtype = true;
                } else if (key == "shape") {
                    if (!j.eat('[')) break;
                    if (!j.eat(']')) {
                        do {
                            uint64_t v;
                            if (!j.num(&v)) break;
                            t.shape.push_back(v);
                        } while (j.eat(','));
                        if (!j.eat(']')) j.ok = false;
                    }
                    have_shape = j.ok;
                } else if (key == "data_offsets") {
                    if (!j.eat('[') || !j.num(&t.begin) || !j.eat(',') || !j.num(&t.end) || !j.eat(']')) j.ok = false;
                    have_off = j.ok;
                } else if (!j.skip()) {
                    break;
                }
            } while (j.ok && j.eat(','));
            if (!j.ok || !j.eat('}') || !have_dtype || !have_shape || !have_off) {
                j.ok = false;
                break;
            }
            uint64_t elems = 1;
            for (uint64_t d : t.shape) elems *= d;
            if (t.end < t.begin || t.end > data_size ||
                (st_dtype_size(t.dtype) && elems * st_dtype_size(t.dtype) != t.end - t.begin)) {
                *err = path + ": tensor '" + name + "' has inconsistent offsets";
                return false;
            }
            tensors_[name] = t;
        } while (j.ok && j.eat(','));
        if (!j.ok || !j.eat('}')) {
            *err = path + ": malformed safetensors header";
            return false;
        }
    }
    return true;
}

const StTensor* StFile::find(const std::string& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

const uint8_t* StFile::bytes(const StTensor& t) const { return data_ + t.begin; }

}  // namespace bh

extern "C" int bh_st_describe(const char* path, const char* name, int* dtype, uint64_t* shape, uint32_t max_rank,
                              uint32_t* rank) {
    if (!path || !name || !dtype || !rank) return bh::fail(BH_ERR_INVALID, "bh_st_describe: null argument");
    bh::StFile f;
    std::string err;
    if (!f.open(path, &err)) return bh::fail(BH_ERR_INVALID, "bh_st_describe: %s", err.c_str());
    const bh::StTensor* t = f.find(name);
    if (!t) return bh::fail(BH_ERR_INVALID, "bh_st_describe: no tensor '%s' in %s", name, path);
    *dtype = t->dtype;
    *rank = (uint32_t)t->shape.size();
    for (uint32_t i = 0; i < *rank && i < max_rank; ++i) shape[i] = t->shape[i];
    return BH_OK;
}
