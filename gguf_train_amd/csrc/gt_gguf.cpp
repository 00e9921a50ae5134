// GGUF reader of libgt_attn.so: the metadata and tensors of a .gguf file, read into host memory
// (the reference's gt_gguf_open / gt_gguf_get_tensor / gt_gguf_kv_*, csrc/gt_ops_extra.cpp:1811-1990)
// or streamed straight into device memory (gt_gguf_get_tensor_device).
//
// File layout (GGUF v2 and v3, little-endian), parsed here without ggml:
//   header      "GGUF", u32 version, u64 n_tensors, u64 n_kv
//   n_kv times  string key, u32 gguf_type, value; an array value is u32 element type, u64 count,
//               then the elements
//   n_tensors   string name, u32 n_dims, u64 ne[n_dims] (innermost dimension first),
//               u32 ggml_type, u64 offset
//   padding to general.alignment (a u32, 32 when absent), then the data section, where tensor i
//   starts at the sum of the sizes of tensors 0..i-1, each padded to the alignment.
// A string is a u64 byte count and the bytes, without a terminator.
//
// The checks are those of ggml's reader (llama.cpp b12283 ggml/src/gguf.cpp, the library the
// reference links): version 2 or 3, no duplicate keys or tensor names, names shorter than 64
// bytes, at most 4 dimensions, ne[0] a multiple of the type's block, offsets in order, the data
// section complete.  A file that fails one of them is "Failed to open GGUF file", the reference's
// message, followed by the reason.
//
// The file stays open until gt_gguf_close; tensor bytes are read (pread) when a tensor is asked
// for, so opening a multi-gigabyte model costs only its header.

#include "gt_internal.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

// enum gguf_type
enum : int {
    KV_U8 = 0, KV_I8, KV_U16, KV_I16, KV_U32, KV_I32, KV_F32, KV_BOOL, KV_STRING, KV_ARRAY, KV_U64, KV_I64, KV_F64,
    KV_NTYPES
};

size_t kv_scalar_size(int t) {
    switch (t) {
        case KV_U8: case KV_I8: case KV_BOOL: return 1;
        case KV_U16: case KV_I16: return 2;
        case KV_U32: case KV_I32: case KV_F32: return 4;
        case KV_U64: case KV_I64: case KV_F64: return 8;
        default: return 0;
    }
}

// ggml tensor types (enum ggml_type): elements per block, bytes per block, name.  A size of 0
// marks an id ggml no longer assigns; such a tensor makes the file unreadable, as in ggml.
struct GgmlType {
    int64_t blck;
    size_t size;
    const char *name;
};
constexpr GgmlType kGgmlTypes[] = {
    {1, 4, "f32"},        {1, 2, "f16"},       {32, 18, "q4_0"},    {32, 20, "q4_1"},     {0, 0, "q4_2"},
    {0, 0, "q4_3"},       {32, 22, "q5_0"},    {32, 24, "q5_1"},    {32, 34, "q8_0"},     {32, 36, "q8_1"},
    {256, 84, "q2_K"},    {256, 110, "q3_K"},  {256, 144, "q4_K"},  {256, 176, "q5_K"},   {256, 210, "q6_K"},
    {256, 292, "q8_K"},   {256, 66, "iq2_xxs"}, {256, 74, "iq2_xs"}, {256, 98, "iq3_xxs"}, {256, 50, "iq1_s"},
    {32, 18, "iq4_nl"},   {256, 110, "iq3_s"}, {256, 82, "iq2_s"},  {256, 136, "iq4_xs"}, {1, 1, "i8"},
    {1, 2, "i16"},        {1, 4, "i32"},       {1, 8, "i64"},       {1, 8, "f64"},        {256, 56, "iq1_m"},
    {1, 2, "bf16"},       {0, 0, "q4_0_4_4"},  {0, 0, "q4_0_4_8"},  {0, 0, "q4_0_8_8"},   {256, 54, "tq1_0"},
    {256, 66, "tq2_0"},   {0, 0, "iq4_nl_4_4"}, {0, 0, "iq4_nl_4_8"}, {0, 0, "iq4_nl_8_8"}, {32, 17, "mxfp4"},
};
constexpr int kGgmlTypeCount = (int)(sizeof(kGgmlTypes) / sizeof(kGgmlTypes[0]));
constexpr int GGML_F32 = 0, GGML_F16 = 1, GGML_I8 = 24, GGML_I16 = 25, GGML_I32 = 26,
              GGML_I64 = 27, GGML_F64 = 28, GGML_BF16 = 30;

const char *ggml_type_name(int t) { return (t >= 0 && t < kGgmlTypeCount) ? kGgmlTypes[t].name : "unknown"; }

// dtype code of a stored ggml type (csrc/gt_ops_extra.cpp gt_ggml_to_dtype): the plain types map
// to their codes, quantized ones to GT_Q_BASE + ggml id.
int dtype_of_ggml(int t) {
    switch (t) {
        case GGML_F32: return GT_F32;
        case GGML_F16: return GT_F16;
        case GGML_BF16: return GT_BF16;
        case GGML_F64: return GT_F64;
        case GGML_I8: return GT_I8;
        case GGML_I16: return GT_I16;
        case GGML_I32: return GT_I32;
        case GGML_I64: return GT_I64;
        default: return GT_Q_BASE + t;
    }
}

constexpr int kMaxName = 64;  // GGML_MAX_NAME, terminator included
constexpr int kMaxDims = 4;   // GGML_MAX_DIMS
constexpr const char *kShapePrefix = "gguf_train.shape.";
constexpr const char *kDtypePrefix = "gguf_train.dtype.";

struct Kv {
    std::string key;
    int type = -1;
    int arr_type = -1;
    uint64_t n = 0;
    std::vector<uint8_t> data;      // a scalar's bytes, or the packed elements of a numeric array
    std::string str;                // a string value
    std::vector<std::string> strs;  // a string array
};

struct TensorInfo {
    std::string name;
    int n_dims = 0;
    int64_t ne[kMaxDims] = {1, 1, 1, 1};
    int type = 0;
    uint64_t offset = 0;  // from the start of the data section
    uint64_t nbytes = 0;
};

// Sequential reads over a file descriptor through a buffer; every read is bounds-checked against
// the file size taken at open.
class Reader {
  public:
    Reader(int fd, uint64_t size) : fd_(fd), size_(size), buf_(1 << 20) {}

    uint64_t tell() const { return pos_; }
    uint64_t left() const { return size_ - pos_; }

    bool read(void *dst, size_t n) {
        if (n > left()) return false;
        auto *out = static_cast<uint8_t *>(dst);
        while (n > 0) {
            if (pos_ < buf_pos_ || pos_ >= buf_pos_ + buf_len_) {
                const size_t want = (size_t)std::min<uint64_t>(buf_.size(), size_ - pos_);
                if (!pread_full(fd_, buf_.data(), want, pos_)) return false;
                buf_pos_ = pos_;
                buf_len_ = want;
            }
            const size_t at = (size_t)(pos_ - buf_pos_);
            const size_t take = std::min(n, buf_len_ - at);
            std::memcpy(out, buf_.data() + at, take);
            out += take;
            pos_ += take;
            n -= take;
        }
        return true;
    }
    template <typename T>
    bool get(T &v) {
        return read(&v, sizeof(T));
    }
    bool string(std::string &s) {
        uint64_t n = 0;
        if (!get(n) || n > left()) return false;
        s.resize((size_t)n);
        return n == 0 || read(&s[0], (size_t)n);
    }

    static bool pread_full(int fd, void *dst, size_t n, uint64_t at) {
        auto *p = static_cast<uint8_t *>(dst);
        while (n > 0) {
            const ssize_t r = ::pread(fd, p, n, (off_t)at);
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) return false;
            p += r;
            n -= (size_t)r;
            at += (uint64_t)r;
        }
        return true;
    }

  private:
    int fd_;
    uint64_t size_;
    uint64_t pos_ = 0;
    std::vector<uint8_t> buf_;
    uint64_t buf_pos_ = 0;
    size_t buf_len_ = 0;
};

}  // namespace

struct gt_gguf_file {
    int fd = -1;
    uint64_t size = 0;
    uint64_t data_offset = 0;
    uint32_t alignment = 32;
    std::vector<Kv> kvs;
    std::unordered_map<std::string, size_t> kv_index;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, size_t> tensor_index;

    ~gt_gguf_file() {
        if (fd >= 0) ::close(fd);
    }
    const Kv *find_kv(const std::string &key) const {
        auto it = kv_index.find(key);
        return it == kv_index.end() ? nullptr : &kvs[it->second];
    }
};

namespace {

bool parse_value(Reader &r, int type, Kv &kv, std::string &err) {
    if (type == KV_STRING) {
        if (!r.string(kv.str)) return err = "truncated string value of '" + kv.key + "'", false;
        return true;
    }
    if (type == KV_ARRAY) {
        uint32_t et = 0;
        uint64_t n = 0;
        if (!r.get(et) || !r.get(n)) return err = "truncated array header of '" + kv.key + "'", false;
        if (et >= KV_NTYPES || et == KV_ARRAY)
            return err = "array '" + kv.key + "' has element type " + std::to_string(et), false;
        kv.arr_type = (int)et;
        kv.n = n;
        if (et == KV_STRING) {
            // each element takes at least its 8-byte length
            if (n > r.left() / 8) return err = "truncated string array '" + kv.key + "'", false;
            kv.strs.resize((size_t)n);
            for (auto &s : kv.strs)
                if (!r.string(s)) return err = "truncated string array '" + kv.key + "'", false;
            return true;
        }
        const size_t es = kv_scalar_size((int)et);
        if (n > r.left() / es) return err = "truncated array '" + kv.key + "'", false;
        kv.data.resize((size_t)(n * es));
        if (n > 0 && !r.read(kv.data.data(), kv.data.size())) return err = "truncated array '" + kv.key + "'", false;
        return true;
    }
    const size_t es = kv_scalar_size(type);
    if (es == 0) return err = "key '" + kv.key + "' has unknown type " + std::to_string(type), false;
    kv.data.resize(es);
    if (!r.read(kv.data.data(), es)) return err = "truncated value of '" + kv.key + "'", false;
    return true;
}

bool parse_file(gt_gguf_file &gf, std::string &err) {
    Reader r(gf.fd, gf.size);
    char magic[4];
    if (!r.read(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return err = "not a GGUF file (bad magic)", false;
    uint32_t version = 0;
    if (!r.get(version)) return err = "truncated header", false;
    if (version == 1) return err = "GGUFv1 is no longer supported", false;
    if (version < 2 || version > 3) return err = "unsupported GGUF version " + std::to_string(version), false;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.get(n_tensors) || !r.get(n_kv)) return err = "truncated header", false;
    // a metadata entry takes at least 12 bytes and a tensor entry at least 24
    if (n_kv > r.left() / 12 || n_tensors > r.left() / 24)
        return err = "truncated file: the header names " + std::to_string(n_kv) + " metadata entries and " +
                     std::to_string(n_tensors) + " tensors, " + std::to_string(r.left()) + " bytes follow", false;

    gf.kvs.resize((size_t)n_kv);
    for (uint64_t i = 0; i < n_kv; ++i) {
        Kv &kv = gf.kvs[(size_t)i];
        uint32_t type = 0;
        if (!r.string(kv.key) || !r.get(type)) return err = "truncated metadata entry " + std::to_string(i), false;
        if (type >= KV_NTYPES) return err = "key '" + kv.key + "' has unknown type " + std::to_string(type), false;
        kv.type = (int)type;
        if (!parse_value(r, kv.type, kv, err)) return false;
        if (!gf.kv_index.emplace(kv.key, (size_t)i).second) return err = "duplicate key '" + kv.key + "'", false;
    }
    if (const Kv *a = gf.find_kv("general.alignment")) {
        if (a->type != KV_U32) return err = "general.alignment is not a u32", false;
        uint32_t v = 0;
        std::memcpy(&v, a->data.data(), 4);
        if (v == 0 || (v & (v - 1)) != 0) return err = "general.alignment " + std::to_string(v) + " is not a power of two", false;
        gf.alignment = v;
    }

    gf.tensors.resize((size_t)n_tensors);
    uint64_t expect = 0;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorInfo &ti = gf.tensors[(size_t)i];
        uint32_t nd = 0, type = 0;
        if (!r.string(ti.name) || !r.get(nd)) return err = "truncated tensor entry " + std::to_string(i), false;
        if (ti.name.size() >= (size_t)kMaxName)
            return err = "tensor name '" + ti.name + "' is " + std::to_string(ti.name.size()) + " bytes long", false;
        if (nd > (uint32_t)kMaxDims)
            return err = "tensor '" + ti.name + "' has " + std::to_string(nd) + " dimensions", false;
        ti.n_dims = (int)nd;
        for (uint32_t d = 0; d < nd; ++d) {
            if (!r.get(ti.ne[d])) return err = "truncated tensor entry '" + ti.name + "'", false;
            if (ti.ne[d] < 0) return err = "tensor '" + ti.name + "' has a negative dimension", false;
        }
        uint64_t off = 0;
        if (!r.get(type) || !r.get(off)) return err = "truncated tensor entry '" + ti.name + "'", false;
        if ((int)type >= kGgmlTypeCount || kGgmlTypes[type].blck == 0)
            return err = "tensor '" + ti.name + "' has unknown ggml type " + std::to_string(type), false;
        ti.type = (int)type;
        ti.offset = off;
        const GgmlType &gt = kGgmlTypes[type];
        if (ti.ne[0] % gt.blck != 0)
            return err = "tensor '" + ti.name + "': ne[0] = " + std::to_string(ti.ne[0]) + " is not a multiple of the " +
                         gt.name + " block size " + std::to_string(gt.blck), false;
        // the element count and byte size must fit int64
        int64_t n = 1;
        for (int d = 0; d < kMaxDims; ++d) {
            if (ti.ne[d] > 0 && n > INT64_MAX / ti.ne[d])
                return err = "tensor '" + ti.name + "' has too many elements", false;
            n *= ti.ne[d];
        }
        const uint64_t blocks = (uint64_t)(n / gt.blck);
        if (blocks > (uint64_t)INT64_MAX / gt.size) return err = "tensor '" + ti.name + "' is too large", false;
        ti.nbytes = blocks * gt.size;
        if (!gf.tensor_index.emplace(ti.name, (size_t)i).second)
            return err = "duplicate tensor name '" + ti.name + "'", false;
        if (ti.offset != expect)
            return err = "tensor '" + ti.name + "' has offset " + std::to_string(ti.offset) + ", expected " +
                         std::to_string(expect), false;
        const uint64_t padded = (ti.nbytes + gf.alignment - 1) / gf.alignment * gf.alignment;
        if (padded > (uint64_t)INT64_MAX - expect) return err = "the data section is too large", false;
        expect += padded;
    }
    const uint64_t hdr = r.tell();
    gf.data_offset = (hdr + gf.alignment - 1) / gf.alignment * gf.alignment;
    if (gf.data_offset > gf.size || expect > gf.size - gf.data_offset)
        return err = "the data section needs " + std::to_string(expect) + " bytes at offset " +
                     std::to_string(gf.data_offset) + ", the file has " + std::to_string(gf.size), false;
    return true;
}

// What gt_gguf_get_tensor makes of a stored tensor: dtype and shape after the reference's
// recorded keys (csrc/gt_ops_extra.cpp:1846-1908), with the same error messages.
struct TensorPlan {
    const TensorInfo *ti = nullptr;
    int dtype = GT_F32;
    std::vector<int64_t> shape;
};

// GGUF keeps at most four dimensions and drops outer dimensions of size one: the natural shape
// reverses ne and keeps dimensions up to the last one above 1 (csrc/gt_ops_extra.cpp:1535-1548).
std::vector<int64_t> natural_shape(const int64_t *ne, bool complex_pairs) {
    int nd = 1;
    for (int i = kMaxDims - 1; i >= 1; --i) {
        if (ne[i] > 1) {
            nd = i + 1;
            break;
        }
    }
    std::vector<int64_t> shape;
    for (int d = nd - 1; d >= 0; --d) shape.push_back(ne[d]);
    if (complex_pairs) {
        if (!shape.empty() && shape.back() == 2) shape.pop_back();
        else shape.clear();
    }
    return shape;
}

bool plan_tensor(const gt_gguf_file *gf, const char *name, TensorPlan &p) {
    auto it = gf->tensor_index.find(name);
    if (it == gf->tensor_index.end()) {
        gt_set_error(std::string("gguf: no tensor named '") + name + "'");
        return false;
    }
    const TensorInfo &ti = gf->tensors[it->second];
    p.ti = &ti;
    const std::string label = std::string("gguf: tensor '") + name + "': ";
    int dt = dtype_of_ggml(ti.type);

    bool cplx = false;
    if (const Kv *rec = gf->find_kv(std::string(kDtypePrefix) + name)) {
        if (rec->type != KV_STRING) {
            gt_set_error(label + "the recorded dtype is not a string");
            return false;
        }
        const std::string &want = rec->str;
        int carrier = -1;
        if (want == "uint8") carrier = GGML_I8, dt = GT_U8;
        else if (want == "bool") carrier = GGML_I8, dt = GT_BOOL;
        else if (want == "complex64") carrier = GGML_F32, dt = GT_C64, cplx = true;
        else if (want == "complex128") carrier = GGML_F64, dt = GT_C128, cplx = true;
        if (carrier != ti.type) {
            gt_set_error(label + "recorded as " + want + " but stored as " + ggml_type_name(ti.type));
            return false;
        }
    }
    int64_t count = 1;
    for (int d = 0; d < kMaxDims; ++d) count *= ti.ne[d];
    if (cplx && count % 2 != 0) {
        gt_set_error(label + "a complex tensor needs an even number of stored values");
        return false;
    }
    const int64_t numel = cplx ? count / 2 : count;

    p.shape = natural_shape(ti.ne, cplx);
    if (const Kv *rec = gf->find_kv(std::string(kShapePrefix) + name)) {
        if (rec->type != KV_ARRAY || rec->arr_type != KV_I64) {
            gt_set_error(label + "the recorded shape is not an int64 array");
            return false;
        }
        if (rec->n > (uint64_t)GT_MAX_DIMS) {
            gt_set_error(label + "the recorded shape has too many dimensions");
            return false;
        }
        p.shape.resize((size_t)rec->n);
        if (rec->n) std::memcpy(p.shape.data(), rec->data.data(), (size_t)rec->n * 8);
    }
    int64_t expect = 1;
    bool valid = true;
    for (int64_t d : p.shape) {
        if (d < 0 || (d > 0 && expect > INT64_MAX / d)) {
            valid = false;
            break;
        }
        expect *= d;
    }
    if (!valid || expect != numel) {
        gt_set_error(label + "the shape does not match the " + std::to_string(numel) + " stored elements");
        return false;
    }
    if (cplx) {
        gt_set_error(label + "complex tensors are not supported by libgt_attn");
        return false;
    }
    if (gt_is_quantized(dt) && dt != GT_Q8_0) {
        gt_set_error(label + "ggml type " + ggml_type_name(ti.type) + " is not supported by libgt_attn (q8_0 only)");
        return false;
    }
    p.dtype = dt;
    return true;
}

// Pinned staging for host -> device streaming: kStageBufs chunks of kStageChunk bytes, one per
// reader thread.  A thread fills its chunk with pread while the copies of the other chunks are in
// flight, so file reads (page-cache copies, which scale with threads) overlap the DMA into HBM.
// The chunks are allocated on first use and kept for the life of the process; one load at a time.
constexpr size_t kStageChunk = 16u << 20;
constexpr int kStageBufs = 8;
struct Staging {
    std::mutex mu;
    void *buf[kStageBufs] = {};
};
Staging &staging() {
    static Staging *s = new Staging();
    return *s;
}

// Copies `nbytes` of the file at `at` into device memory `dst` of device `dev` on `stream`;
// returns when the copies are complete.  Chunk c is read by thread c % nthreads.
bool stream_to_device(int fd, uint64_t at, uint64_t nbytes, void *dst, int dev, hipStream_t stream,
                      const std::string &label) {
    if (nbytes == 0) return true;
    const uint64_t nchunks = (nbytes + kStageChunk - 1) / kStageChunk;
    const int nthreads = (int)std::min<uint64_t>(kStageBufs, nchunks);
    Staging &sg = staging();
    std::lock_guard<std::mutex> lock(sg.mu);
    for (int w = 0; w < nthreads; ++w)
        if (!sg.buf[w] &&
            !gt_hip_check(hipHostMalloc(&sg.buf[w], kStageChunk, hipHostMallocDefault), "hipHostMalloc (gguf staging)"))
            return false;

    struct Worker {
        hipEvent_t ev = nullptr;
        bool used = false;
        std::string err;  // errors are per thread: each worker keeps its own message
    };
    std::vector<Worker> wk((size_t)nthreads);
    auto run = [&](int w) {
        Worker &me = wk[(size_t)w];
        auto fail = [&](const std::string &m) { me.err = m.empty() ? "HIP error" : m; };
        if (hipSetDevice(dev) != hipSuccess || hipEventCreateWithFlags(&me.ev, hipEventDisableTiming) != hipSuccess)
            return fail(label + "cannot set up the staging copy");
        for (uint64_t c = (uint64_t)w; c < nchunks; c += (uint64_t)nthreads) {
            const uint64_t off = c * kStageChunk;
            const size_t n = (size_t)std::min<uint64_t>(kStageChunk, nbytes - off);
            // the copy that last read this chunk must be finished before pread overwrites it
            if (me.used && !gt_hip_check(hipEventSynchronize(me.ev), "hipEventSynchronize")) return fail(gt_last_error());
            if (!Reader::pread_full(fd, sg.buf[w], n, at + off))
                return fail(label + "reading the file failed (was it changed after it was opened?)");
            if (!gt_hip_check(hipMemcpyAsync((char *)dst + off, sg.buf[w], n, hipMemcpyHostToDevice, stream),
                              "hipMemcpyAsync") ||
                !gt_hip_check(hipEventRecord(me.ev, stream), "hipEventRecord"))
                return fail(gt_last_error());
            me.used = true;
        }
    };
    std::vector<std::thread> threads;
    for (int w = 1; w < nthreads; ++w) threads.emplace_back(run, w);
    run(0);
    for (auto &t : threads) t.join();
    // no copy may still read the staging buffers once the lock is released
    std::string err;
    for (Worker &w : wk) {
        if (w.used && hipEventSynchronize(w.ev) != hipSuccess && w.err.empty()) w.err = label + "a staging copy failed";
        if (w.ev) (void)hipEventDestroy(w.ev);
        if (err.empty()) err = w.err;
    }
    if (!err.empty()) {
        gt_set_error(err);
        return false;
    }
    return true;
}

}  // namespace

extern "C" gt_gguf_file *gt_gguf_open(const char *path) {
    if (!path) {
        gt_set_error("Failed to open GGUF file: NULL path");
        return nullptr;
    }
    auto *gf = new gt_gguf_file();
    std::string err;
    gf->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    struct stat sb;
    if (gf->fd < 0) {
        err = std::string(path) + ": " + std::strerror(errno);
    } else if (::fstat(gf->fd, &sb) != 0 || !S_ISREG(sb.st_mode)) {
        err = std::string(path) + " is not a regular file";
    } else {
        gf->size = (uint64_t)sb.st_size;
        parse_file(*gf, err);
    }
    if (!err.empty()) {
        delete gf;
        gt_set_error("Failed to open GGUF file: " + err);
        return nullptr;
    }
    return gf;
}

extern "C" void gt_gguf_close(gt_gguf_file *gf) { delete gf; }

extern "C" int64_t gt_gguf_n_tensors(const gt_gguf_file *gf) { return gf ? (int64_t)gf->tensors.size() : 0; }

extern "C" const char *gt_gguf_tensor_name(const gt_gguf_file *gf, int64_t idx) {
    if (!gf || idx < 0 || idx >= (int64_t)gf->tensors.size()) return nullptr;
    return gf->tensors[(size_t)idx].name.c_str();
}

extern "C" gt_tensor *gt_gguf_get_tensor(const gt_gguf_file *gf, const char *name, int dequantize_f32) {
    if (!gf || !name) {
        gt_set_error("gguf: NULL file or name");
        return nullptr;
    }
    TensorPlan p;
    if (!plan_tensor(gf, name, p)) return nullptr;
    gt_tensor *raw = gt_new_tensor((int)p.shape.size(), p.shape.data(), p.dtype, GT_DEV_CPU, 0);
    if (!raw) return nullptr;
    if (p.ti->nbytes > 0 && !Reader::pread_full(gf->fd, gt_data(raw), (size_t)p.ti->nbytes, gf->data_offset + p.ti->offset)) {
        gt_tensor_free(raw);
        gt_set_error(std::string("gguf: tensor '") + name + "': reading the file failed (was it changed after it was opened?)");
        return nullptr;
    }
    if (dequantize_f32 && gt_is_quantized(p.dtype)) {
        gt_tensor *f32 = gt_tensor_to_dtype(raw, GT_F32);
        gt_tensor_free(raw);
        return f32;
    }
    return raw;
}

extern "C" gt_tensor *gt_gguf_get_tensor_device(const gt_gguf_file *gf, const char *name, int dequantize_f32,
                                                int device_index) {
    if (!gf || !name) {
        gt_set_error("gguf: NULL file or name");
        return nullptr;
    }
    TensorPlan p;
    if (!plan_tensor(gf, name, p)) return nullptr;
    if (!gt_device_ok(device_index)) return nullptr;
    gt_tensor *raw = gt_new_tensor((int)p.shape.size(), p.shape.data(), p.dtype, GT_DEV_CUDA, device_index);
    if (!raw) return nullptr;
    const std::string label = std::string("gguf: tensor '") + name + "': ";
    if (!stream_to_device(gf->fd, gf->data_offset + p.ti->offset, p.ti->nbytes, gt_data(raw), device_index,
                          gt_stream(), label)) {
        gt_tensor_free(raw);
        return nullptr;
    }
    if (dequantize_f32 && gt_is_quantized(p.dtype)) {
        gt_tensor *f32 = gt_dequantize(raw, GT_F32);  // on the device, same stream
        gt_tensor_free(raw);
        return f32;
    }
    return raw;
}

extern "C" int64_t gt_gguf_n_kv(const gt_gguf_file *gf) { return gf ? (int64_t)gf->kvs.size() : 0; }

static const Kv *kv_at(const gt_gguf_file *gf, int64_t idx) {
    return (gf && idx >= 0 && idx < (int64_t)gf->kvs.size()) ? &gf->kvs[(size_t)idx] : nullptr;
}

extern "C" const char *gt_gguf_kv_key(const gt_gguf_file *gf, int64_t idx) {
    const Kv *kv = kv_at(gf, idx);
    return kv ? kv->key.c_str() : nullptr;
}

extern "C" int gt_gguf_kv_type(const gt_gguf_file *gf, int64_t idx) {
    const Kv *kv = kv_at(gf, idx);
    return kv ? kv->type : -1;
}

// The value as text, snprintf-style: the full length is returned and a result >= buf_len means
// the text was cut short (csrc/gt_ops_extra.cpp:1936-1970).  Floats are printed with 17
// significant digits, which read back as the same double (a float32 as the double it widens to).
extern "C" int gt_gguf_kv_val_str(const gt_gguf_file *gf, int64_t idx, char *buf, int buf_len) {
    const Kv *kv = kv_at(gf, idx);
    if (!kv) return -1;
    char *out = (buf && buf_len > 0) ? buf : nullptr;
    const size_t cap = out ? (size_t)buf_len : 0;
    auto val = [&](auto zero) {
        decltype(zero) v;
        std::memcpy(&v, kv->data.data(), sizeof(v));
        return v;
    };
    switch (kv->type) {
        case KV_STRING: {
            const size_t len = kv->str.size();
            if (out) {
                const size_t ncopy = std::min(len, cap - 1);
                std::memcpy(out, kv->str.data(), ncopy);
                out[ncopy] = '\0';
            }
            return len > (size_t)INT_MAX ? INT_MAX : (int)len;
        }
        case KV_U8: return std::snprintf(out, cap, "%u", (unsigned)val(uint8_t()));
        case KV_I8: return std::snprintf(out, cap, "%d", (int)val(int8_t()));
        case KV_U16: return std::snprintf(out, cap, "%u", (unsigned)val(uint16_t()));
        case KV_I16: return std::snprintf(out, cap, "%d", (int)val(int16_t()));
        case KV_U32: return std::snprintf(out, cap, "%u", val(uint32_t()));
        case KV_I32: return std::snprintf(out, cap, "%d", val(int32_t()));
        case KV_F32: return std::snprintf(out, cap, "%.17g", (double)val(float()));
        case KV_U64: return std::snprintf(out, cap, "%llu", (unsigned long long)val(uint64_t()));
        case KV_I64: return std::snprintf(out, cap, "%lld", (long long)val(int64_t()));
        case KV_F64: return std::snprintf(out, cap, "%.17g", val(double()));
        case KV_BOOL: return std::snprintf(out, cap, "%s", val(int8_t()) ? "true" : "false");
        case KV_ARRAY: return std::snprintf(out, cap, "<array len=%llu>", (unsigned long long)kv->n);
        default:
            if (out) out[0] = '\0';
            return 0;
    }
}

extern "C" int gt_gguf_kv_arr_type(const gt_gguf_file *gf, int64_t idx) {
    const Kv *kv = kv_at(gf, idx);
    return (kv && kv->type == KV_ARRAY) ? kv->arr_type : -1;
}

extern "C" int64_t gt_gguf_kv_arr_n(const gt_gguf_file *gf, int64_t idx) {
    const Kv *kv = kv_at(gf, idx);
    return (kv && kv->type == KV_ARRAY) ? (int64_t)kv->n : -1;
}

extern "C" const void *gt_gguf_kv_arr_data(const gt_gguf_file *gf, int64_t idx) {
    const Kv *kv = kv_at(gf, idx);
    if (!kv || kv->type != KV_ARRAY || kv->arr_type == KV_STRING) return nullptr;
    // an empty array still has a (non-null) address
    static const uint64_t kEmpty = 0;
    return kv->data.empty() ? (const void *)&kEmpty : (const void *)kv->data.data();
}

extern "C" const char *gt_gguf_kv_arr_str(const gt_gguf_file *gf, int64_t idx, int64_t i) {
    const Kv *kv = kv_at(gf, idx);
    if (!kv || kv->type != KV_ARRAY || kv->arr_type != KV_STRING) return nullptr;
    if (i < 0 || (uint64_t)i >= kv->n) return nullptr;
    return kv->strs[(size_t)i].c_str();
}
