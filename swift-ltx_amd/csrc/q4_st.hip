// q4_st.hip -- safetensors reader for the 4-bit path's weights (host code).
//
// The file format swift-ltx reads (SafeTensorsFile, SafeTensors.swift:41-89):
// an 8-byte little-endian header length, a JSON object mapping tensor names to
// {"dtype", "shape", "data_offsets": [begin, end]} (offsets relative to the
// data region that follows the header), an optional "__metadata__" entry, then
// the raw tensor bytes.  Entries with dtypes outside F32/F16/BF16/I8/U8/I32/U32
// are skipped, as the reference does.  Unlike the reference, a tensor whose
// byte range does not match its shape and dtype, or that runs past the end of
// the file, makes the file invalid instead of being read out of bounds.
//
// Reads go straight from the file into device memory through two pinned
// staging buffers (pread of chunk i+1 overlaps the copy of chunk i), the
// analogue of readTensorIntoBuffer (SafeTensors.swift:175-186) with a HIP
// device buffer as the destination.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "q4_common.hpp"
#include "q4_launch.hpp"
#include "swiftltx_q4.h"

namespace sltx {
namespace {

// ---- minimal JSON (objects, arrays, strings, numbers, true/false/null) ----

struct JVal {
    enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
    double num = 0.0;
    bool is_int = false;
    long long inum = 0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
};

class JParser {
public:
    JParser(const char* s, size_t n) : p_(s), end_(s + n) {}
    bool parse(JVal& v) {
        if (!value(v, 0)) return false;
        ws();
        return p_ == end_;
    }

private:
    const char* p_;
    const char* end_;
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w) {
        const size_t n = std::strlen(w);
        if ((size_t)(end_ - p_) < n || std::memcmp(p_, w, n) != 0) return false;
        p_ += n;
        return true;
    }
    static int hexv(char c) {
        if (c >= '0' && c <= '9') return c - '0';
        if (c >= 'a' && c <= 'f') return c - 'a' + 10;
        if (c >= 'A' && c <= 'F') return c - 'A' + 10;
        return -1;
    }
    bool string(std::string& out) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if ((unsigned char)c < 0x20) return false;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p_ >= end_) return false;
            c = *p_++;
            switch (c) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    if (end_ - p_ < 4) return false;
                    unsigned cp = 0;
                    for (int i = 0; i < 4; ++i) {
                        const int h = hexv(p_[i]);
                        if (h < 0) return false;
                        cp = cp * 16 + (unsigned)h;
                    }
                    p_ += 4;
                    // UTF-8 encode (surrogate pairs kept as two 3-byte units)
                    if (cp < 0x80) {
                        out.push_back((char)cp);
                    } else if (cp < 0x800) {
                        out.push_back((char)(0xC0 | (cp >> 6)));
                        out.push_back((char)(0x80 | (cp & 0x3F)));
                    } else {
                        out.push_back((char)(0xE0 | (cp >> 12)));
                        out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
                        out.push_back((char)(0x80 | (cp & 0x3F)));
                    }
                    break;
                }
                default: return false;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool number(JVal& v) {
        const char* s = p_;
        if (p_ < end_ && *p_ == '-') ++p_;
        bool frac = false;
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' ||
                             *p_ == 'E' || *p_ == '+' || *p_ == '-')) {
            if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') frac = true;
            ++p_;
        }
        if (p_ == s) return false;
        const std::string t(s, p_);
        char* e = nullptr;
        v.kind = JVal::kNum;
        v.num = std::strtod(t.c_str(), &e);
        if (e != t.c_str() + t.size()) return false;
        if (!frac) {
            errno = 0;
            v.inum = std::strtoll(t.c_str(), &e, 10);
            v.is_int = errno == 0 && e == t.c_str() + t.size();
        }
        return true;
    }
    bool value(JVal& v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = JVal::kObj;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                JVal child;
                if (!value(child, depth + 1)) return false;
                v.obj.emplace_back(std::move(k), std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = JVal::kArr;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                JVal child;
                if (!value(child, depth + 1)) return false;
                v.arr.push_back(std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            v.kind = JVal::kStr;
            return string(v.str);
        }
        if (lit("true")) {
            v.kind = JVal::kBool;
            v.num = 1;
            return true;
        }
        if (lit("false")) {
            v.kind = JVal::kBool;
            return true;
        }
        if (lit("null")) {
            v.kind = JVal::kNull;
            return true;
        }
        return number(v);
    }
};

const JVal* jget(const JVal& o, const char* key) {
    for (const auto& kv : o.obj)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

// TensorDType (SafeTensors.swift:15-31): names and element sizes.
struct DtypeName {
    const char* name;
    int code;
    int size;
};
constexpr DtypeName kDtypes[] = {{"F32", SLTX_ST_F32, 4}, {"F16", SLTX_ST_F16, 2},
                                 {"BF16", SLTX_ST_BF16, 2}, {"I8", SLTX_ST_I8, 1},
                                 {"U8", SLTX_ST_U8, 1},   {"I32", SLTX_ST_I32, 4},
                                 {"U32", SLTX_ST_U32, 4}};

constexpr size_t kMaxHeader = 100u << 20;
constexpr size_t kChunk = 16u << 20;   // staging chunk for device reads

}  // namespace

struct StFile {
    std::string path;
    int fd = -1;
    uint64_t file_size = 0;
    uint64_t data_offset = 0;
    std::vector<std::string> names;              // sorted
    std::map<std::string, sltx_st_info> tensors;
    std::mutex mu;                               // serialises reads (staging buffers)
    void* staging[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int staging_dev = -1;

    ~StFile() {
        for (int i = 0; i < 2; ++i) {
            if (done[i]) (void)hipEventDestroy(done[i]);
            if (staging[i]) (void)hipHostFree(staging[i]);
        }
        if (fd >= 0) ::close(fd);
    }
};

namespace {

int parse_header(StFile& f, const std::string& hdr) {
    JVal root;
    JParser jp(hdr.data(), hdr.size());
    if (!jp.parse(root) || root.kind != JVal::kObj)
        return set_error(kErrInvalid, "%s: header is not a JSON object", f.path.c_str());
    const uint64_t data_size = f.file_size - f.data_offset;
    for (const auto& kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const JVal& t = kv.second;
        if (t.kind != JVal::kObj) continue;
        const JVal* dt = jget(t, "dtype");
        const JVal* sh = jget(t, "shape");
        const JVal* of = jget(t, "data_offsets");
        if (!dt || dt->kind != JVal::kStr || !sh || sh->kind != JVal::kArr || !of ||
            of->kind != JVal::kArr || of->arr.size() != 2)
            continue;   // the reference skips malformed entries
        const DtypeName* d = nullptr;
        for (const auto& c : kDtypes)
            if (dt->str == c.name) d = &c;
        if (!d) continue;   // unknown dtype: skipped, as in the reference
        sltx_st_info info;
        std::memset(&info, 0, sizeof(info));
        info.dtype = d->code;
        if (sh->arr.size() > 8)
            return set_error(kErrInvalid, "%s: tensor '%s' has more than 8 dimensions",
                             f.path.c_str(), kv.first.c_str());
        info.ndim = (int32_t)sh->arr.size();
        unsigned __int128 elems = 1;
        for (size_t i = 0; i < sh->arr.size(); ++i) {
            const JVal& e = sh->arr[i];
            if (e.kind != JVal::kNum || !e.is_int || e.inum < 0)
                return set_error(kErrInvalid, "%s: tensor '%s' has a bad shape", f.path.c_str(),
                                 kv.first.c_str());
            info.shape[i] = e.inum;
            elems *= (unsigned __int128)e.inum;
        }
        const JVal& b = of->arr[0];
        const JVal& e = of->arr[1];
        if (b.kind != JVal::kNum || e.kind != JVal::kNum || !b.is_int || !e.is_int || b.inum < 0 ||
            e.inum < b.inum || (uint64_t)e.inum > data_size)
            return set_error(kErrInvalid, "%s: tensor '%s' has data_offsets outside the file",
                             f.path.c_str(), kv.first.c_str());
        info.offset = (uint64_t)b.inum;
        info.nbytes = (uint64_t)(e.inum - b.inum);
        if (elems * (unsigned __int128)d->size != (unsigned __int128)info.nbytes)
            return set_error(kErrInvalid,
                             "%s: tensor '%s': %llu bytes do not match its shape and dtype",
                             f.path.c_str(), kv.first.c_str(), (unsigned long long)info.nbytes);
        // A repeated name is ambiguous (which entry holds the data?): the
        // file is rejected rather than keeping one of them.
        if (!f.tensors.emplace(kv.first, info).second)
            return set_error(kErrInvalid, "%s: duplicate tensor name '%s' in the header",
                             f.path.c_str(), kv.first.c_str());
        f.names.push_back(kv.first);
    }
    std::sort(f.names.begin(), f.names.end());
    return kOk;
}

bool read_all(int fd, void* dst, size_t n, uint64_t off) {
    char* p = static_cast<char*>(dst);
    while (n > 0) {
        const ssize_t r = ::pread(fd, p, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        p += r;
        n -= (size_t)r;
        off += (uint64_t)r;
    }
    return true;
}

const sltx_st_info* lookup(const StFile* f, const char* fn, const char* name) {
    if (!f || !name) {
        set_error(kErrInvalid, "%s: null argument", fn);
        return nullptr;
    }
    auto it = f->tensors.find(name);
    if (it == f->tensors.end()) {
        set_error(kErrInvalid, "%s: tensor '%s' not found in %s", fn, name, f->path.c_str());
        return nullptr;
    }
    return &it->second;
}

// Pinned staging buffers and events for the current device (created on the
// first device read).
int ensure_staging(StFile& f, const char* fn) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(kErrHip, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
    if (f.staging[0] && f.staging_dev == dev) return kOk;
    for (int i = 0; i < 2; ++i) {
        if (f.done[i]) (void)hipEventDestroy(f.done[i]);
        if (f.staging[i]) (void)hipHostFree(f.staging[i]);
        f.done[i] = nullptr;
        f.staging[i] = nullptr;
    }
    for (int i = 0; i < 2; ++i) {
        if ((e = hipHostMalloc(&f.staging[i], kChunk, hipHostMallocDefault)) != hipSuccess ||
            (e = hipEventCreateWithFlags(&f.done[i], hipEventDisableTiming)) != hipSuccess)
            return set_error(kErrHip, "%s: staging allocation: %s", fn, hipGetErrorString(e));
    }
    f.staging_dev = dev;
    return kOk;
}

// Copies nbytes of tensor data from file offset off to device dst, converting
// each chunk with cvt (bytes in -> bytes out, out/in size ratio `grow`) when
// given.  Returns after every copy has completed.
template <typename Cvt>
int read_to_device(StFile& f, const char* fn, uint64_t off, uint64_t nbytes, char* dst, int grow,
                   Cvt cvt, hipStream_t st) {
    int rc = ensure_staging(f, fn);
    if (rc != kOk) return rc;
    const size_t in_chunk = kChunk / (size_t)grow;
    std::vector<char> tmp(grow > 1 ? in_chunk : 0);
    uint64_t done_in = 0;
    int i = 0;
    while (done_in < nbytes) {
        const size_t n = (size_t)std::min<uint64_t>(in_chunk, nbytes - done_in);
        const int b = i & 1;
        hipError_t e = hipEventSynchronize(f.done[b]);   // the copy that last used buffer b
        if (e != hipSuccess) return set_error(kErrHip, "%s: %s", fn, hipGetErrorString(e));
        char* stage = static_cast<char*>(f.staging[b]);
        if (!read_all(f.fd, grow > 1 ? tmp.data() : stage, n, f.data_offset + off + done_in))
            return set_error(kErrInvalid, "%s: read error in %s", fn, f.path.c_str());
        if (grow > 1) cvt(tmp.data(), stage, n);
        e = hipMemcpyAsync(dst + done_in * grow, stage, n * grow, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipEventRecord(f.done[b], st);
        if (e != hipSuccess) return set_error(kErrHip, "%s: %s", fn, hipGetErrorString(e));
        done_in += n;
        ++i;
    }
    for (int b = 0; b < 2; ++b) {
        const hipError_t e = hipEventSynchronize(f.done[b]);
        if (e != hipSuccess) return set_error(kErrHip, "%s: %s", fn, hipGetErrorString(e));
    }
    return kOk;
}

float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {   // subnormal: normalise
            int e = -1;
            do {
                man <<= 1;
                ++e;
            } while (!(man & 0x400));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FF) << 13);
        }
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace
}  // namespace sltx

using namespace sltx;

extern "C" {

int sltx_st_open(const char* path, sltx_st_file** out) {
    const char* fn = "sltx_st_open";
    if (!path || !out) return set_error(kErrInvalid, "%s: null argument", fn);
    *out = nullptr;
    std::unique_ptr<StFile> f(new StFile);
    f->path = path;
    f->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) return set_error(kErrInvalid, "%s: cannot open %s: %s", fn, path, std::strerror(errno));
    struct stat sb;
    if (fstat(f->fd, &sb) != 0) return set_error(kErrInvalid, "%s: cannot stat %s", fn, path);
    f->file_size = (uint64_t)sb.st_size;
    uint64_t hlen = 0;
    unsigned char le[8];
    if (f->file_size < 8 || !read_all(f->fd, le, 8, 0))
        return set_error(kErrInvalid, "%s: %s is too short for a safetensors header", fn, path);
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | le[i];
    if (hlen > kMaxHeader || hlen > f->file_size - 8)
        return set_error(kErrInvalid, "%s: %s: header length %llu is invalid", fn, path,
                         (unsigned long long)hlen);
    std::string hdr((size_t)hlen, '\0');
    if (!read_all(f->fd, &hdr[0], (size_t)hlen, 8))
        return set_error(kErrInvalid, "%s: cannot read the header of %s", fn, path);
    f->data_offset = 8 + hlen;
    const int rc = parse_header(*f, hdr);
    if (rc != kOk) return rc;
    *out = reinterpret_cast<sltx_st_file*>(f.release());
    return kOk;
}

void sltx_st_close(sltx_st_file* file) { delete reinterpret_cast<StFile*>(file); }

int sltx_st_num_tensors(const sltx_st_file* file) {
    if (!file) return set_error(kErrInvalid, "sltx_st_num_tensors: null file");
    return (int)reinterpret_cast<const StFile*>(file)->names.size();
}

const char* sltx_st_name(const sltx_st_file* file, int32_t index) {
    const StFile* f = reinterpret_cast<const StFile*>(file);
    if (!f || index < 0 || (size_t)index >= f->names.size()) return nullptr;
    return f->names[(size_t)index].c_str();
}

int sltx_st_info_of(const sltx_st_file* file, const char* name, sltx_st_info* out) {
    const sltx_st_info* info = lookup(reinterpret_cast<const StFile*>(file), "sltx_st_info_of", name);
    if (!info) return kErrInvalid;
    if (!out) return set_error(kErrInvalid, "sltx_st_info_of: null out");
    *out = *info;
    return kOk;
}

int sltx_st_read_host(sltx_st_file* file, const char* name, void* dst, uint64_t capacity) {
    const char* fn = "sltx_st_read_host";
    StFile* f = reinterpret_cast<StFile*>(file);
    const sltx_st_info* info = lookup(f, fn, name);
    if (!info) return kErrInvalid;
    if (!dst && info->nbytes) return set_error(kErrInvalid, "%s: null destination", fn);
    if (capacity < info->nbytes)
        return set_error(kErrInvalid, "%s: '%s' needs %llu bytes, capacity %llu", fn, name,
                         (unsigned long long)info->nbytes, (unsigned long long)capacity);
    if (!read_all(f->fd, dst, (size_t)info->nbytes, f->data_offset + info->offset))
        return set_error(kErrInvalid, "%s: read error in %s", fn, f->path.c_str());
    return kOk;
}

int sltx_st_read_device(sltx_st_file* file, const char* name, void* dst, uint64_t capacity,
                        void* stream) {
    const char* fn = "sltx_st_read_device";
    StFile* f = reinterpret_cast<StFile*>(file);
    const sltx_st_info* info = lookup(f, fn, name);
    if (!info) return kErrInvalid;
    if (!dst && info->nbytes) return set_error(kErrInvalid, "%s: null destination", fn);
    if (capacity < info->nbytes)
        return set_error(kErrInvalid, "%s: '%s' needs %llu bytes, capacity %llu", fn, name,
                         (unsigned long long)info->nbytes, (unsigned long long)capacity);
    if (info->nbytes == 0) return kOk;
    std::lock_guard<std::mutex> lk(f->mu);
    return read_to_device(*f, fn, info->offset, info->nbytes, static_cast<char*>(dst), 1,
                          [](const char*, char*, size_t) {}, static_cast<hipStream_t>(stream));
}

int sltx_st_read_device_f32(sltx_st_file* file, const char* name, float* dst, uint64_t count,
                            void* stream) {
    const char* fn = "sltx_st_read_device_f32";
    StFile* f = reinterpret_cast<StFile*>(file);
    const sltx_st_info* info = lookup(f, fn, name);
    if (!info) return kErrInvalid;
    int esize = 0;
    if (info->dtype == SLTX_ST_F32) esize = 4;
    else if (info->dtype == SLTX_ST_F16 || info->dtype == SLTX_ST_BF16) esize = 2;
    else return set_error(kErrInvalid, "%s: '%s' is not a floating-point tensor", fn, name);
    const uint64_t n = info->nbytes / (uint64_t)esize;
    if (count < n)
        return set_error(kErrInvalid, "%s: '%s' has %llu elements, capacity %llu", fn, name,
                         (unsigned long long)n, (unsigned long long)count);
    if (!dst && n) return set_error(kErrInvalid, "%s: null destination", fn);
    if (n == 0) return kOk;
    std::lock_guard<std::mutex> lk(f->mu);
    hipStream_t st = static_cast<hipStream_t>(stream);
    char* d = reinterpret_cast<char*>(dst);
    if (esize == 4)
        return read_to_device(*f, fn, info->offset, info->nbytes, d, 1,
                              [](const char*, char*, size_t) {}, st);
    // loadFloat / the bf16 branch of loadRaw (ModelWeights.swift:66-75, :96-108)
    if (info->dtype == SLTX_ST_F16)
        return read_to_device(*f, fn, info->offset, info->nbytes, d, 2,
                              [](const char* in, char* out, size_t nb) {
                                  const uint16_t* s = reinterpret_cast<const uint16_t*>(in);
                                  float* o = reinterpret_cast<float*>(out);
                                  for (size_t i = 0; i < nb / 2; ++i) o[i] = f16_bits_to_f32(s[i]);
                              },
                              st);
    return read_to_device(*f, fn, info->offset, info->nbytes, d, 2,
                          [](const char* in, char* out, size_t nb) {
                              const uint16_t* s = reinterpret_cast<const uint16_t*>(in);
                              uint32_t* o = reinterpret_cast<uint32_t*>(out);
                              for (size_t i = 0; i < nb / 2; ++i) o[i] = (uint32_t)s[i] << 16;
                          },
                          st);
}

}  // extern "C"
