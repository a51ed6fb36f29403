// GGUF v3 reader and whole-file upload (include/qk_gguf.h).  Parsing follows the GGUF v3 layout the
// reference reads (qwen_cpu/gguf.h:106-175); the upload mirrors qwen_cuda/qwen.cpp:737-761 with
// the T16 repack in place of the reference's Q8_0/Q6_K row repack.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../include/qk_gguf.h"
#include "qk_internal.h"

struct qk_gguf {
    struct Tensor {
        std::string name;
        uint32_t type = 0;
        int32_t ndims = 0;
        int64_t dims[4] = {1, 1, 1, 1};
        uint64_t offset = 0;  // from the file start
        uint64_t nbytes = 0;
        uint32_t layout = QK_LAYOUT_GGUF;
    };
    std::vector<uint8_t> host;  // the file; released by the upload
    uint64_t size = 0;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> index;
    std::unordered_map<std::string, double> kv_num;
    std::unordered_map<std::string, std::string> kv_str;
    uint8_t* dev = nullptr;  // device copy of the whole file
};

namespace {

// Bounds-checked little-endian cursor over the file bytes.
struct Cursor {
    const uint8_t* p;
    const uint8_t* end;
    bool ok = true;
    bool need(uint64_t n) {
        if (!ok || (uint64_t)(end - p) < n) ok = false;
        return ok;
    }
    template <class T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p, sizeof(T));
            p += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return {};
        std::string s((const char*)p, (size_t)n);
        p += n;
        return s;
    }
};

// GGUF value types 0..12: uint8, int8, uint16, int16, uint32, int32, float32, bool, string, array,
// uint64, int64, float64.
constexpr uint64_t VALUE_BYTES[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};

bool skip_value(Cursor& c, uint32_t t, int depth = 0) {
    if (t > 12 || depth > 4) return c.ok = false;
    if (t == 8) {
        c.str();
        return c.ok;
    }
    if (t == 9) {
        const uint32_t et = c.get<uint32_t>();
        const uint64_t n = c.get<uint64_t>();
        if (et > 12) return c.ok = false;
        if (et == 8 || et == 9) {
            for (uint64_t i = 0; i < n && c.ok; i++) skip_value(c, et, depth + 1);
            return c.ok;
        }
        if (n > (uint64_t)(c.end - c.p) / VALUE_BYTES[et]) return c.ok = false;
        c.p += n * VALUE_BYTES[et];
        return true;
    }
    if (c.need(VALUE_BYTES[t])) c.p += VALUE_BYTES[t];
    return c.ok;
}

double read_number(Cursor& c, uint32_t t) {
    switch (t) {
        case 0: return c.get<uint8_t>();
        case 1: return c.get<int8_t>();
        case 2: return c.get<uint16_t>();
        case 3: return c.get<int16_t>();
        case 4: return c.get<uint32_t>();
        case 5: return c.get<int32_t>();
        case 6: return c.get<float>();
        case 7: return c.get<uint8_t>();
        case 10: return (double)c.get<uint64_t>();
        case 11: return (double)c.get<int64_t>();
        case 12: return c.get<double>();
    }
    c.ok = false;
    return 0.0;
}

int read_file(const char* path, std::vector<uint8_t>& buf) {
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) return QK_E_IO;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 0) {
        ::close(fd);
        return QK_E_IO;
    }
    buf.resize((size_t)st.st_size);
    for (size_t off = 0; off < buf.size();) {
        const size_t want = std::min(buf.size() - off, (size_t)1 << 30);
        const ssize_t n = pread(fd, buf.data() + off, want, (off_t)off);
        if (n <= 0) {
            ::close(fd);
            return QK_E_IO;
        }
        off += (size_t)n;
    }
    ::close(fd);
    return QK_OK;
}

bool repackable(const qk_gguf::Tensor& t) {
    const bool quant = t.type == QK_T_Q8_0 || t.type == QK_T_Q4_K || t.type == QK_T_Q5_K || t.type == QK_T_Q6_K;
    return quant && t.ndims == 2 && t.dims[0] % 256 == 0 && t.dims[1] % 16 == 0 && t.dims[0] <= INT32_MAX &&
           t.dims[1] <= INT32_MAX;
}

}  // namespace

extern "C" {

int qk_gguf_open(const char* path, qk_gguf** out) {
    if (!path || !out) return QK_E_NULL;
    *out = nullptr;
    qk_gguf* f = new qk_gguf();
    int rc = read_file(path, f->host);
    if (rc != QK_OK) {
        delete f;
        return rc;
    }
    f->size = f->host.size();
    Cursor c{f->host.data(), f->host.data() + f->host.size()};
    rc = QK_E_FORMAT;
    if (c.get<uint32_t>() != 0x46554747u || c.get<uint32_t>() != 3) {  // "GGUF", version 3
        delete f;
        return rc;
    }
    const uint64_t nt = c.get<uint64_t>(), nkv = c.get<uint64_t>();
    for (uint64_t i = 0; i < nkv && c.ok; i++) {
        const std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        if (t == 8) f->kv_str[key] = c.str();
        else if (t == 9) skip_value(c, t);
        else f->kv_num[key] = read_number(c, t);
    }
    for (uint64_t i = 0; i < nt && c.ok; i++) {
        qk_gguf::Tensor t;
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (nd < 1 || nd > 4) c.ok = false;
        for (uint32_t d = 0; d < nd && c.ok; d++) {
            const uint64_t v = c.get<uint64_t>();
            if (v < 1 || v > (uint64_t)INT32_MAX) c.ok = false;  // every dimension in [1, 2^31)
            t.dims[d] = (int64_t)v;
        }
        t.ndims = (int32_t)nd;
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();  // relative to the data start until fixed below
        f->tensors.push_back(t);
    }
    if (!c.ok) {
        delete f;
        return rc;
    }
    const auto al = f->kv_num.find("general.alignment");
    const uint64_t align = al != f->kv_num.end() && al->second >= 1 ? (uint64_t)al->second : 32;
    const uint64_t data_start = ((uint64_t)(c.p - f->host.data()) + align - 1) / align * align;
    for (size_t i = 0; i < f->tensors.size(); i++) {
        qk_gguf::Tensor& t = f->tensors[i];
        t.offset += data_start;
        // rows and bytes with overflow checks: a crafted header cannot wrap them into a small size
        uint64_t numel = 1, rb = 0, nbytes = 0;
        bool bad = false;
        for (int d = 1; d < t.ndims; d++) bad = bad || __builtin_mul_overflow(numel, (uint64_t)t.dims[d], &numel);
        if (qk_row_bytes(t.type, t.dims[0], &rb) == QK_OK) bad = bad || __builtin_mul_overflow(rb, numel, &nbytes);
        t.nbytes = nbytes;
        if (bad || t.offset > f->size || t.nbytes > f->size - t.offset) {  // data past the end of the file
            delete f;
            return rc;
        }
        f->index[t.name] = (int64_t)i;
    }
    *out = f;
    return QK_OK;
}

void qk_gguf_close(qk_gguf* f) {
    if (!f) return;
    if (f->dev) (void)hipFree(f->dev);
    delete f;
}

int qk_gguf_tensor_count(const qk_gguf* f, int64_t* count) {
    if (!f || !count) return QK_E_NULL;
    *count = (int64_t)f->tensors.size();
    return QK_OK;
}

int qk_gguf_tensor_info(const qk_gguf* f, int64_t i, const char** name, uint32_t* type, int32_t* ndims,
                        int64_t dims[4], uint64_t* file_offset, uint64_t* nbytes) {
    if (!f) return QK_E_NULL;
    if (i < 0 || i >= (int64_t)f->tensors.size()) return QK_E_RANGE;
    const qk_gguf::Tensor& t = f->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (type) *type = t.type;
    if (ndims) *ndims = t.ndims;
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = t.dims[d];
    if (file_offset) *file_offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return QK_OK;
}

int qk_gguf_find(const qk_gguf* f, const char* name, int64_t* index) {
    if (!f || !name || !index) return QK_E_NULL;
    const auto it = f->index.find(name);
    if (it == f->index.end()) return QK_E_NOTFOUND;
    *index = it->second;
    return QK_OK;
}

int qk_gguf_kv_num(const qk_gguf* f, const char* key, double* value) {
    if (!f || !key || !value) return QK_E_NULL;
    const auto it = f->kv_num.find(key);
    if (it == f->kv_num.end()) return QK_E_NOTFOUND;
    *value = it->second;
    return QK_OK;
}

int qk_gguf_kv_str(const qk_gguf* f, const char* key, const char** value) {
    if (!f || !key || !value) return QK_E_NULL;
    const auto it = f->kv_str.find(key);
    if (it == f->kv_str.end()) return QK_E_NOTFOUND;
    *value = it->second.c_str();
    return QK_OK;
}

int qk_gguf_upload(qk_gguf* f, qk_stream_t stream) {
    if (!f) return QK_E_NULL;
    if (f->dev) return QK_OK;  // set only once an upload has completed
    if (f->host.empty()) return QK_E_RANGE;
    const hipStream_t s = (hipStream_t)stream;
    uint8_t* dev = nullptr;
    if (hipMalloc((void**)&dev, f->size) != hipSuccess) return QK_E_HIP;
    // in-place T16 repack through one scratch buffer of the largest eligible tensor
    uint64_t scratch_bytes = 0;
    for (const auto& t : f->tensors)
        if (repackable(t)) scratch_bytes = std::max(scratch_bytes, t.nbytes);
    uint8_t* scratch = nullptr;
    int rc = QK_OK;
    if (hipMemcpyAsync(dev, f->host.data(), f->size, hipMemcpyHostToDevice, s) != hipSuccess ||
        (scratch_bytes && hipMalloc((void**)&scratch, scratch_bytes) != hipSuccess))
        rc = QK_E_HIP;
    for (auto& t : f->tensors) {
        if (rc != QK_OK) break;
        if (!repackable(t)) continue;
        uint8_t* at = dev + t.offset;
        uint64_t rb = 0;
        (void)qk_row_bytes(t.type, t.dims[0], &rb);
        if (hipMemcpyAsync(scratch, at, t.nbytes, hipMemcpyDeviceToDevice, s) != hipSuccess ||
            qk::launch_repack(scratch, at, (int)t.type, (int)t.dims[0], (int)t.dims[1], rb, 0, s) != 0)
            rc = QK_E_HIP;
    }
    if (hipStreamSynchronize(s) != hipSuccess && rc == QK_OK) rc = QK_E_HIP;
    if (scratch) (void)hipFree(scratch);
    if (rc != QK_OK) {  // nothing half-uploaded survives: a later call starts over
        (void)hipFree(dev);
        return rc;
    }
    for (auto& t : f->tensors)
        if (repackable(t)) t.layout = QK_LAYOUT_T16;
    f->dev = dev;
    f->host.clear();
    f->host.shrink_to_fit();
    return QK_OK;
}

int qk_gguf_weight(const qk_gguf* f, const char* name, qk_weight* w) {
    if (!f || !name || !w) return QK_E_NULL;
    if (!f->dev) return QK_E_RANGE;  // not uploaded
    const auto it = f->index.find(name);
    if (it == f->index.end()) return QK_E_NOTFOUND;
    const qk_gguf::Tensor& t = f->tensors[(size_t)it->second];
    if (t.ndims != 2 || t.dims[0] > INT32_MAX || t.dims[1] > INT32_MAX) return QK_E_SHAPE;
    return qk_weight_view(f->dev + t.offset, t.type, (int32_t)t.dims[0], (int32_t)t.dims[1], t.layout, w);
}

}  // extern "C"
