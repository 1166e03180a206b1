// moa_ckpt.hip -- the checkpoint reader (include/moa_ckpt.h): the reference's on-disk format,
// one safetensors file (FO/src/host/load.rs), mapped read-only, its header parsed once, tensors
// validated as load.rs validates them and copied to device memory through pinned staging.
//
// File layout (the safetensors format): an unsigned 64-bit little-endian header length n, n bytes
// of JSON -- an object mapping each tensor name to {"dtype", "shape", "data_offsets": [begin, end]},
// plus an optional "__metadata__" object of strings -- then the data section; offsets are relative
// to its start.
//
// Host code only: no kernels. Device copies use two pinned buffers of kStageBytes. While the DMA
// engine copies one to the device, host threads fill the other from the mapping.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/moa_ckpt.h"
#include "moa_internal.h"

struct moa_ckpt {
    struct Tensor {
        std::string dtype;
        std::vector<int64_t> shape;
        uint64_t begin = 0, end = 0;
    };
    std::string path;
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    const uint8_t* data = nullptr;  // start of the data section
    size_t data_size = 0;
    std::vector<std::string> names;                 // header order
    std::unordered_map<std::string, Tensor> tensors;
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int stage_device = -1;
};

namespace moa {
namespace {

constexpr uint64_t kMaxHeader = 100ull << 20;  // the format's own limit on the JSON header
constexpr size_t kStageBytes = 32u << 20;

int err(int code, const std::string& msg) { return set_error(code, msg.c_str()); }

// Element size of a safetensors dtype; 0 for a dtype this reader does not size.
size_t dtype_size(const std::string& d) {
    if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E4M3" || d == "F8_E5M2" || d == "F8_E8M0") return 1;
    if (d == "U16" || d == "I16" || d == "F16" || d == "BF16") return 2;
    if (d == "U32" || d == "I32" || d == "F32") return 4;
    if (d == "U64" || d == "I64" || d == "F64") return 8;
    return 0;
}

// ------------------------------------------------------------------- JSON (the header's subset)
// A recursive-descent reader of objects, arrays, strings, integers and literals. Numbers other
// than non-negative integers are skipped as values (only shapes and offsets are read).
class Json {
  public:
    Json(const char* p, size_t n) : p_(p), e_(p + n) {}
    std::string error;

    bool header(moa_ckpt* c) {
        ws();
        if (!take('{')) return fail("header is not a JSON object");
        ws();
        if (take('}')) return end();
        for (;;) {
            std::string key;
            ws();
            if (!string(key)) return false;
            ws();
            if (!take(':')) return fail("expected ':' after \"" + key + "\"");
            ws();
            if (key == "__metadata__") {
                if (!skip_value(0)) return false;
            } else {
                if (c->tensors.count(key)) return fail("tensor \"" + key + "\" appears twice");
                moa_ckpt::Tensor t;
                if (!tensor(key, t)) return false;
                c->names.push_back(key);
                c->tensors.emplace(key, std::move(t));
            }
            ws();
            if (take(',')) continue;
            if (take('}')) return end();
            return fail("expected ',' or '}' in the header object");
        }
    }

  private:
    const char* p_;
    const char* e_;

    bool fail(const std::string& m) {
        if (error.empty()) error = m;
        return false;
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool take(char ch) {
        if (p_ < e_ && *p_ == ch) {
            ++p_;
            return true;
        }
        return false;
    }
    bool end() {
        ws();
        // the format pads the header with spaces; anything else after the object is an error
        if (p_ != e_) return fail("trailing bytes after the header object");
        return true;
    }
    bool string(std::string& out) {
        if (!take('"')) return fail("expected a string");
        out.clear();
        while (p_ < e_ && *p_ != '"') {
            char ch = *p_++;
            if ((unsigned char)ch < 0x20) return fail("control character in a string");
            if (ch != '\\') {
                out.push_back(ch);
                continue;
            }
            if (p_ >= e_) break;
            ch = *p_++;
            switch (ch) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    uint32_t cp = 0;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                        uint32_t lo = 0;
                        if (!(take('\\') && take('u') && hex4(lo)) || lo < 0xDC00 || lo >= 0xE000)
                            return fail("unpaired surrogate in a string");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(cp, out);
                    break;
                }
                default: return fail("bad escape in a string");
            }
        }
        if (!take('"')) return fail("unterminated string");
        return true;
    }
    bool hex4(uint32_t& v) {
        if (e_ - p_ < 4) return fail("short \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char ch = *p_++;
            v <<= 4;
            if (ch >= '0' && ch <= '9') v |= ch - '0';
            else if (ch >= 'a' && ch <= 'f') v |= ch - 'a' + 10;
            else if (ch >= 'A' && ch <= 'F') v |= ch - 'A' + 10;
            else return fail("bad \\u escape");
        }
        return true;
    }
    static void utf8(uint32_t cp, std::string& out) {
        if (cp < 0x80) out.push_back((char)cp);
        else if (cp < 0x800) {
            out.push_back((char)(0xC0 | (cp >> 6)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            out.push_back((char)(0xE0 | (cp >> 12)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            out.push_back((char)(0xF0 | (cp >> 18)));
            out.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
        }
    }
    bool uint(uint64_t& v) {
        if (p_ >= e_ || *p_ < '0' || *p_ > '9') return fail("expected a non-negative integer");
        v = 0;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = (uint64_t)(*p_++ - '0');
            if (v > (UINT64_MAX - d) / 10) return fail("integer overflow");
            v = v * 10 + d;
        }
        if (p_ < e_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E')) return fail("expected an integer");
        return true;
    }
    bool uint_array(std::vector<uint64_t>& out) {
        if (!take('[')) return fail("expected an array");
        ws();
        if (take(']')) return true;
        for (;;) {
            ws();
            uint64_t v = 0;
            if (!uint(v)) return false;
            out.push_back(v);
            ws();
            if (take(',')) continue;
            if (take(']')) return true;
            return fail("expected ',' or ']' in an array");
        }
    }
    bool tensor(const std::string& name, moa_ckpt::Tensor& t) {
        if (!take('{')) return fail("entry \"" + name + "\" is not an object");
        bool has_dtype = false, has_shape = false, has_offsets = false;
        ws();
        if (!take('}')) {
            for (;;) {
                std::string key;
                ws();
                if (!string(key)) return false;
                ws();
                if (!take(':')) return fail("expected ':' in entry \"" + name + "\"");
                ws();
                if (key == "dtype") {
                    if (!string(t.dtype)) return false;
                    has_dtype = true;
                } else if (key == "shape") {
                    std::vector<uint64_t> s;
                    if (!uint_array(s)) return false;
                    for (uint64_t d : s) {
                        if (d > (uint64_t)INT64_MAX) return fail("dimension too large in \"" + name + "\"");
                        t.shape.push_back((int64_t)d);
                    }
                    has_shape = true;
                } else if (key == "data_offsets") {
                    std::vector<uint64_t> o;
                    if (!uint_array(o)) return false;
                    if (o.size() != 2) return fail("data_offsets of \"" + name + "\" is not [begin, end]");
                    t.begin = o[0];
                    t.end = o[1];
                    has_offsets = true;
                } else if (!skip_value(0)) {
                    return false;
                }
                ws();
                if (take(',')) continue;
                if (take('}')) break;
                return fail("expected ',' or '}' in entry \"" + name + "\"");
            }
        }
        if (!has_dtype || !has_shape || !has_offsets)
            return fail("entry \"" + name + "\" lacks dtype, shape or data_offsets");
        return true;
    }
    bool skip_value(int depth) {
        if (depth > 64) return fail("header nested too deeply");
        ws();
        if (p_ >= e_) return fail("unexpected end of header");
        const char ch = *p_;
        if (ch == '"') {
            std::string s;
            return string(s);
        }
        if (ch == '{' || ch == '[') {
            const char close = ch == '{' ? '}' : ']';
            ++p_;
            ws();
            if (take(close)) return true;
            for (;;) {
                ws();
                if (ch == '{') {
                    std::string k;
                    if (!string(k)) return false;
                    ws();
                    if (!take(':')) return fail("expected ':'");
                }
                if (!skip_value(depth + 1)) return false;
                ws();
                if (take(',')) continue;
                if (take(close)) return true;
                return fail("unterminated object or array");
            }
        }
        // number or literal
        const char* s = p_;
        while (p_ < e_ && (std::strchr("+-.eE0123456789", *p_) || std::isalpha((unsigned char)*p_))) ++p_;
        if (p_ == s) return fail("unexpected character in header");
        const std::string tok(s, p_);
        if (std::isalpha((unsigned char)tok[0]) && tok != "true" && tok != "false" && tok != "null")
            return fail("unknown literal in header");
        return true;
    }
};

// The header is JSON, so UTF-8: every byte sequence must be a well-formed UTF-8 character (no
// overlong forms, no surrogates, nothing above U+10FFFF), as a JSON reader of the format requires.
bool valid_utf8(const uint8_t* p, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t b = p[i];
        if (b < 0x80) { ++i; continue; }
        int len;
        uint32_t cp;
        if ((b & 0xE0) == 0xC0) { len = 2; cp = b & 0x1F; }
        else if ((b & 0xF0) == 0xE0) { len = 3; cp = b & 0x0F; }
        else if ((b & 0xF8) == 0xF0) { len = 4; cp = b & 0x07; }
        else return false;
        if (i + len > n) return false;
        for (int k = 1; k < len; ++k) {
            if ((p[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (p[i + k] & 0x3F);
        }
        static const uint32_t kMin[5] = {0, 0, 0x80, 0x800, 0x10000};
        if (cp < kMin[len] || cp > 0x10FFFF || (cp >= 0xD800 && cp < 0xE000)) return false;
        i += len;
    }
    return true;
}

int parse(moa_ckpt* c) {
    if (c->size < 8) return err(MOA_ERROR_FORMAT, c->path + ": shorter than the 8-byte header length");
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = (n << 8) | c->map[i];
    if (n > kMaxHeader) return err(MOA_ERROR_FORMAT, c->path + ": header length " + std::to_string(n) + " too large");
    if (n > c->size - 8) return err(MOA_ERROR_FORMAT, c->path + ": header runs past the end of the file");
    if (!valid_utf8(c->map + 8, (size_t)n)) return err(MOA_ERROR_FORMAT, c->path + ": header is not valid UTF-8");
    Json j(reinterpret_cast<const char*>(c->map + 8), (size_t)n);
    if (!j.header(c)) return err(MOA_ERROR_FORMAT, c->path + ": " + j.error);
    c->data = c->map + 8 + n;
    c->data_size = c->size - 8 - (size_t)n;
    for (const auto& name : c->names) {
        const moa_ckpt::Tensor& t = c->tensors.at(name);
        if (t.shape.size() > 8) return err(MOA_ERROR_FORMAT, name + ": more than 8 dimensions");
        if (t.begin > t.end || t.end > c->data_size)
            return err(MOA_ERROR_FORMAT, name + ": data_offsets outside the data section");
        const size_t es = dtype_size(t.dtype);
        if (es) {
            uint64_t numel = 1;
            for (int64_t d : t.shape) {
                if (d != 0 && numel > UINT64_MAX / (uint64_t)d) return err(MOA_ERROR_FORMAT, name + ": shape overflows");
                numel *= (uint64_t)d;
            }
            if (numel > UINT64_MAX / es || numel * es != t.end - t.begin)
                return err(MOA_ERROR_FORMAT, name + ": byte range does not match dtype and shape");
        }
    }
    return MOA_SUCCESS;
}

std::string shape_str(const std::vector<int64_t>& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

// The tensor `name` if it has `dtype` and `shape`; else nullptr with the error recorded in *code.
const moa_ckpt::Tensor* expect(const moa_ckpt* c, const char* name, const char* dtype,
                               const std::vector<int64_t>& shape, int* code) {
    if (!c || !name) {
        *code = err(MOA_ERROR_INVALID_VALUE, "null checkpoint handle or tensor name");
        return nullptr;
    }
    auto it = c->tensors.find(name);
    if (it == c->tensors.end()) {
        *code = err(MOA_ERROR_NOT_FOUND, std::string(name) + ": not in " + c->path);
        return nullptr;
    }
    const moa_ckpt::Tensor& t = it->second;
    if (t.dtype != dtype || t.shape != shape) {
        *code = err(MOA_ERROR_FORMAT, std::string(name) + " is " + t.dtype + " " + shape_str(t.shape) + ", expected " +
                                          dtype + " " + shape_str(shape));
        return nullptr;
    }
    *code = MOA_SUCCESS;
    return &t;
}

int hip_err(hipError_t e, const char* what) { return err(MOA_ERROR_HIP, std::string(what) + ": " + hipGetErrorString(e)); }

void free_stage(moa_ckpt* c) {
    for (int i = 0; i < 2; ++i) {
        if (c->done[i]) {
            (void)hipEventSynchronize(c->done[i]);
            (void)hipEventDestroy(c->done[i]);
            c->done[i] = nullptr;
        }
        if (c->stage[i]) {
            (void)hipHostFree(c->stage[i]);
            c->stage[i] = nullptr;
        }
    }
    c->stage_device = -1;
}

// Fills a staging buffer from the mapping with kCopyThreads threads: one thread's memcpy out of
// the page cache (about 30 GB/s) is slower than the host-to-device DMA it feeds.
constexpr size_t kCopyThreads = 4;
void stage_copy(uint8_t* dst, const uint8_t* src, size_t len) {
    if (len < (4u << 20)) {
        std::memcpy(dst, src, len);
        return;
    }
    const size_t part = (len / kCopyThreads + 4095) & ~(size_t)4095;
    std::thread th[kCopyThreads - 1];
    for (size_t k = 1; k < kCopyThreads; ++k) {
        const size_t a = std::min(len, k * part), b = std::min(len, (k + 1) * part);
        th[k - 1] = std::thread([=] { if (b > a) std::memcpy(dst + a, src + a, b - a); });
    }
    std::memcpy(dst, src, std::min(len, part));
    for (auto& x : th) x.join();
}

// Copies n bytes from host memory `src` to device memory `dst`, staged through the handle's two
// pinned buffers; returns once the last copy has completed.
int copy_to_device(moa_ckpt* c, const void* src, uint64_t n, void* dst, hipStream_t s) {
    if (!dst) return err(MOA_ERROR_INVALID_VALUE, "null destination");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_err(e, "hipGetDevice");
    if (c->stage_device != dev) {
        free_stage(c);
        for (int i = 0; i < 2; ++i) {
            e = hipHostMalloc(&c->stage[i], kStageBytes, hipHostMallocDefault);
            if (e != hipSuccess) {
                free_stage(c);
                return hip_err(e, "hipHostMalloc (checkpoint staging)");
            }
            e = hipEventCreateWithFlags(&c->done[i], hipEventDisableTiming);
            if (e != hipSuccess) {
                free_stage(c);
                return hip_err(e, "hipEventCreateWithFlags");
            }
        }
        c->stage_device = dev;
    }
    const uint8_t* from = static_cast<const uint8_t*>(src);
    uint8_t* to = static_cast<uint8_t*>(dst);
    int i = 0;
    for (uint64_t off = 0; off < n; off += kStageBytes, i ^= 1) {
        const size_t len = (size_t)std::min<uint64_t>(kStageBytes, n - off);
        e = hipEventSynchronize(c->done[i]);  // the buffer's previous copy has finished
        if (e != hipSuccess) return hip_err(e, "hipEventSynchronize");
        stage_copy(static_cast<uint8_t*>(c->stage[i]), from + off, len);
        e = hipMemcpyAsync(to + off, c->stage[i], len, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return hip_err(e, "hipMemcpyAsync (checkpoint)");
        e = hipEventRecord(c->done[i], s);
        if (e != hipSuccess) return hip_err(e, "hipEventRecord");
    }
    for (int k = 0; k < 2; ++k) {
        e = hipEventSynchronize(c->done[k]);
        if (e != hipSuccess) return hip_err(e, "hipEventSynchronize");
    }
    return MOA_SUCCESS;
}

int load(moa_ckpt* c, const char* name, const char* dtype, const std::vector<int64_t>& shape, void* dst, void* stream) {
    int code = 0;
    const moa_ckpt::Tensor* t = expect(c, name, dtype, shape, &code);
    if (!t) return code;
    return copy_to_device(c, c->data + t->begin, t->end - t->begin, dst, static_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace moa

using moa::err;

extern "C" {

int moa_ckpt_open(const char* path, moa_ckpt** out) {
    if (!path || !out) return err(MOA_ERROR_INVALID_VALUE, "null path or output handle");
    *out = nullptr;
    auto* c = new moa_ckpt();
    c->path = path;
    c->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (c->fd < 0) {
        delete c;
        return err(MOA_ERROR_IO, std::string(path) + ": " + std::strerror(errno));
    }
    struct stat st;
    if (fstat(c->fd, &st) != 0 || st.st_size < 0) {
        const int en = errno;
        ::close(c->fd);
        delete c;
        return err(MOA_ERROR_IO, std::string(path) + ": " + std::strerror(en));
    }
    c->size = (size_t)st.st_size;
    if (c->size) {
        void* m = mmap(nullptr, c->size, PROT_READ, MAP_PRIVATE, c->fd, 0);
        if (m == MAP_FAILED) {
            const int en = errno;
            ::close(c->fd);
            delete c;
            return err(MOA_ERROR_IO, std::string(path) + ": mmap: " + std::strerror(en));
        }
        c->map = static_cast<const uint8_t*>(m);
    }
    const int code = moa::parse(c);
    if (code != MOA_SUCCESS) {
        moa_ckpt_close(c);
        return code;
    }
    *out = c;
    return MOA_SUCCESS;
}

int moa_ckpt_close(moa_ckpt* c) {
    if (!c) return MOA_SUCCESS;
    moa::free_stage(c);
    if (c->map) munmap(const_cast<uint8_t*>(c->map), c->size);
    if (c->fd >= 0) ::close(c->fd);
    delete c;
    return MOA_SUCCESS;
}

int moa_ckpt_count(const moa_ckpt* c, int* count) {
    if (!c || !count) return err(MOA_ERROR_INVALID_VALUE, "null argument");
    *count = (int)c->names.size();
    return MOA_SUCCESS;
}

int moa_ckpt_name(const moa_ckpt* c, int index, const char** name) {
    if (!c || !name) return err(MOA_ERROR_INVALID_VALUE, "null argument");
    if (index < 0 || index >= (int)c->names.size()) return err(MOA_ERROR_INVALID_VALUE, "tensor index out of range");
    *name = c->names[index].c_str();
    return MOA_SUCCESS;
}

int moa_ckpt_info(const moa_ckpt* c, const char* name, const char** dtype, int64_t* shape, int* ndim,
                  uint64_t* nbytes) {
    if (!c || !name) return err(MOA_ERROR_INVALID_VALUE, "null checkpoint handle or tensor name");
    auto it = c->tensors.find(name);
    if (it == c->tensors.end()) return err(MOA_ERROR_NOT_FOUND, std::string(name) + ": not in " + c->path);
    const moa_ckpt::Tensor& t = it->second;
    if (dtype) *dtype = t.dtype.c_str();
    if (ndim) *ndim = (int)t.shape.size();
    if (shape)
        for (size_t i = 0; i < t.shape.size(); ++i) shape[i] = t.shape[i];
    if (nbytes) *nbytes = t.end - t.begin;
    return MOA_SUCCESS;
}

int moa_ckpt_read(const moa_ckpt* c, const char* name, void* host_dst, uint64_t nbytes) {
    if (!c || !name || (!host_dst && nbytes)) return err(MOA_ERROR_INVALID_VALUE, "null argument");
    auto it = c->tensors.find(name);
    if (it == c->tensors.end()) return err(MOA_ERROR_NOT_FOUND, std::string(name) + ": not in " + c->path);
    const moa_ckpt::Tensor& t = it->second;
    if (nbytes != t.end - t.begin)
        return err(MOA_ERROR_INVALID_VALUE, std::string(name) + ": holds " + std::to_string(t.end - t.begin) +
                                                " bytes, not " + std::to_string(nbytes));
    if (nbytes) std::memcpy(host_dst, c->data + t.begin, nbytes);
    return MOA_SUCCESS;
}

int moa_ckpt_load_bf16(moa_ckpt* c, const char* name, const int64_t* shape, int ndim, void* dst, void* stream) {
    if (ndim < 0 || ndim > 8 || (ndim && !shape)) return err(MOA_ERROR_INVALID_VALUE, "bad expected shape");
    return moa::load(c, name, "BF16", std::vector<int64_t>(shape, shape + ndim), dst, stream);
}

int moa_ckpt_load_bf16_column(moa_ckpt* c, const char* name, int64_t n, void* dst, void* stream) {
    return moa::load(c, name, "BF16", {n, 1}, dst, stream);
}

int moa_ckpt_load_f8(moa_ckpt* c, const char* name, int64_t rows, int64_t cols, void* dst, void* stream) {
    return moa::load(c, name, "F8_E4M3", {rows, cols}, dst, stream);
}

int moa_ckpt_load_f4(moa_ckpt* c, const char* name, int64_t rows, int64_t cols, void* dst, void* stream) {
    if (cols % 2) return err(MOA_ERROR_INVALID_VALUE, "E2M1 column count must be even");
    return moa::load(c, name, "U8", {rows, cols / 2}, dst, stream);
}

int moa_ckpt_load_scalar_bf16(moa_ckpt* c, const char* name, void* dst, void* stream) {
    int code = 0;
    const moa_ckpt::Tensor* t = moa::expect(c, name, "BF16", {1}, &code);
    if (!t) return code;
    uint16_t v8[8];
    uint16_t v;
    std::memcpy(&v, c->data + t->begin, 2);
    for (auto& x : v8) x = v;
    return moa::copy_to_device(c, v8, sizeof(v8), dst, static_cast<hipStream_t>(stream));
}

int moa_ckpt_global_scale(const moa_ckpt* c, const char* name, float* reciprocal) {
    if (!reciprocal) return err(MOA_ERROR_INVALID_VALUE, "null output");
    if (!c || !name) return err(MOA_ERROR_INVALID_VALUE, "null checkpoint handle or tensor name");
    auto it = c->tensors.find(name);
    if (it == c->tensors.end()) return err(MOA_ERROR_NOT_FOUND, std::string(name) + ": not in " + c->path);
    const moa_ckpt::Tensor& t = it->second;
    // read_f32 (load.rs:162-168): any shape, as long as it is one F32 value
    if (t.dtype != "F32" || t.end - t.begin != 4)
        return err(MOA_ERROR_FORMAT, std::string(name) + " is " + t.dtype + ", not a scalar f32 tensor");
    float g;
    std::memcpy(&g, c->data + t.begin, 4);
    if (g == 0.0f || !std::isfinite(g))
        return err(MOA_ERROR_FORMAT, "invalid NVFP4 global scale " + std::string(name) + ": " + std::to_string(g));
    *reciprocal = 1.0f / g;
    return MOA_SUCCESS;
}

int moa_ckpt_load_global_scale(moa_ckpt* c, const char* name, void* dst, void* stream) {
    float r = 0.0f;
    const int code = moa_ckpt_global_scale(c, name, &r);
    if (code != MOA_SUCCESS) return code;
    return moa::copy_to_device(c, &r, sizeof(r), dst, static_cast<hipStream_t>(stream));
}

}  // extern "C"
