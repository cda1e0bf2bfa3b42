// safetensors header parsing and file mapping (host code).  The checks follow what
// SafeTensors::deserialize rejects before the reference's loader sees a tensor
// (src/engine/loader.rs:36-46): a header that does not fit the file, malformed JSON,
// offsets outside the data region or reversed, and a byte length that does not
// match the shape and dtype.
#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>

#include "../../include/ppocr_rechead.h"
#include "json.hpp"

namespace ppocr {

int fail(int code, const std::string& msg);  // api.hip: sets the thread's last error

namespace {

// Errors of the model file are PPOCR_ERR_MODEL, in the form of OcrError::SafeTensorsError.
int st_fail(const std::string& msg) { return fail(PPOCR_ERR_MODEL, "SafeTensors: " + msg); }

}  // namespace

size_t st_dtype_size(const std::string& d) {
    if (d == "F64" || d == "I64" || d == "U64") return 8;
    if (d == "F32" || d == "I32" || d == "U32") return 4;
    if (d == "F16" || d == "BF16" || d == "I16" || d == "U16") return 2;
    if (d == "I8" || d == "U8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    return 0;
}

StFile::~StFile() {
    if (map_) munmap(map_, size_);
}

int StFile::open(const char* path) {
    if (!path) return st_fail("null path");
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(PPOCR_ERR_MODEL, std::string("Model: failed to read model file ") + path + ": " + strerror(errno));
    struct stat stt;
    if (fstat(fd, &stt) != 0) {
        ::close(fd);
        return fail(PPOCR_ERR_MODEL, std::string("Model: failed to stat model file ") + path);
    }
    size_ = (size_t)stt.st_size;
    if (size_ < 8) {
        ::close(fd);
        return st_fail("file too short for a header");
    }
    map_ = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map_ == MAP_FAILED) {
        map_ = nullptr;
        return fail(PPOCR_ERR_MODEL, std::string("Model: failed to map model file ") + path);
    }
    const uint8_t* base = static_cast<const uint8_t*>(map_);
    uint64_t hlen = 0;
    for (int b = 7; b >= 0; --b) hlen = (hlen << 8) | base[b];
    if (hlen > size_ - 8) return st_fail("header length " + std::to_string(hlen) + " exceeds the file");
    const uint8_t* data0 = base + 8 + hlen;
    const size_t data_bytes = size_ - 8 - (size_t)hlen;

    Json js{reinterpret_cast<const char*>(base + 8), reinterpret_cast<const char*>(data0), {}};
    auto bad = [&](const std::string& what) { return st_fail("invalid header: " + (js.err.empty() ? what : js.err)); };
    if (!js.expect('{')) return bad("");
    std::vector<StTensor> ts;
    if (!js.peek('}')) {
        do {
            std::string key;
            if (!js.string(&key) || !js.expect(':')) return bad("");
            if (key == "__metadata__") {
                // a map of strings (the reference's bundles keep the model graph here)
                JVal md;
                if (!js.value(&md)) return bad("");
                if (md.kind != JVal::kObj) return st_fail("invalid header: __metadata__ is not an object");
                for (auto& kv : md.obj)
                    if (kv.second.kind == JVal::kStr) metadata_.push_back({kv.first, std::move(kv.second.s)});
                continue;
            }
            StTensor t;
            t.name = key;
            bool have_dtype = false, have_shape = false, have_off = false;
            std::vector<int64_t> off;
            if (!js.expect('{')) return bad("");
            if (!js.peek('}')) {
                do {
                    std::string f;
                    if (!js.string(&f) || !js.expect(':')) return bad("");
                    if (f == "dtype") {
                        if (!js.string(&t.dtype)) return bad("");
                        have_dtype = true;
                    } else if (f == "shape") {
                        if (!js.int_array(&t.shape)) return bad("");
                        have_shape = true;
                    } else if (f == "data_offsets") {
                        if (!js.int_array(&off)) return bad("");
                        have_off = true;
                    } else if (!js.skip()) {
                        return bad("");
                    }
                } while (js.peek(',') && ++js.p);
            }
            if (!js.expect('}')) return bad("");
            if (!have_dtype || !have_shape || !have_off || off.size() != 2)
                return st_fail("tensor '" + key + "': missing dtype, shape or data_offsets");
            const size_t es = st_dtype_size(t.dtype);
            if (es == 0) return st_fail("tensor '" + key + "': unknown dtype " + t.dtype);
            if (off[0] < 0 || off[1] < off[0] || (uint64_t)off[1] > data_bytes)
                return st_fail("tensor '" + key + "': data offsets outside the data region");
            uint64_t count = 1;
            for (int64_t d : t.shape) {
                if (d < 0 || (d > 0 && count > UINT64_MAX / (uint64_t)d))
                    return st_fail("tensor '" + key + "': invalid shape");
                count *= (uint64_t)d;
            }
            t.bytes = (size_t)(off[1] - off[0]);
            if (count > UINT64_MAX / es || count * es != (uint64_t)t.bytes)
                return st_fail("tensor '" + key + "': " + std::to_string(t.bytes) + " bytes is not the size of its shape and dtype");
            t.data = data0 + off[0];
            ts.push_back(std::move(t));
        } while (js.peek(',') && ++js.p);
    }
    if (!js.expect('}')) return bad("");
    js.ws();
    if (js.p != js.end) return st_fail("invalid header: trailing bytes");
    tensors_ = std::move(ts);
    return PPOCR_OK;
}

const StTensor* StFile::find(const char* name) const {
    if (!name) return nullptr;
    for (const StTensor& t : tensors_)
        if (t.name == name) return &t;
    return nullptr;
}

}  // namespace ppocr
