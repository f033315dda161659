// Weight I/O in the reference's protobuf format: a reader and writer of CollectionLibraryData
// (engine/ml/src/main/proto/collections.proto:1-27) on the protobuf wire format, host only.
//
// Wire format (public protobuf encoding): every field is a varint key (field << 3 | wire type)
// followed by a varint (type 0), 8 bytes (type 1), a varint length + bytes (type 2) or 4 bytes
// (type 5).  Repeated scalars arrive packed (one type-2 run, the proto3 default and what both
// the Java and the Python writers emit) or one element per key; both are accepted, and fields
// this schema does not know are skipped.  A sub-message field that repeats is merged, as the
// protobuf runtime does (repeated fields append, scalars keep the last value).
//
// Files are memory-mapped for the dictionary's lifetime; a packed data_32 run is kept as a
// pointer into the mapping (little-endian fp32 is the wire layout), so a multi-GB weight file
// is neither copied nor decoded on the host.
//
// Loading follows StateDictionary.loadWeights (engine/ml/.../ml/StateDictionary.java:119-150):
// every file of the directory whose name does not start with '.', each parsed on its own; a parse
// failure skips the rest of that file with a warning and keeps what it had yielded; entries with
// an empty shape are dropped (CollectionEncoder.decode, engine/ml/.../persist/assets/
// CollectionEncoder.java:126-140); later keys replace earlier ones.  Files are read in name
// order (Java's File.listFiles order is unspecified).  Values: `data` (double) when present,
// else `data_32` (CollectionDataMemory.java:51,73).
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/ar_state_dict.h"

void ar_set_error(const char* fmt, ...);

namespace {

struct Mapping {
    void* base = nullptr;
    size_t size = 0;
    ~Mapping() {
        if (base && size) munmap(base, size);
    }
};

// Values of one repeated field: packed runs pointing into a mapping, or owned storage.
template <typename T>
struct Values {
    std::vector<std::pair<const unsigned char*, int64_t>> runs;  // (little-endian bytes, element count)
    std::vector<T> own;                                           // values added one by one / put()
    int64_t count() const {
        int64_t n = (int64_t)own.size();
        for (auto& r : runs) n += r.second;
        return n;
    }
};

struct Tensor {
    std::vector<int32_t> dims;
    int axis = 0;
    Values<double> f64;
    Values<float> f32;
    bool has_f64() const { return f64.count() > 0; }
    int64_t count() const { return has_f64() ? f64.count() : f32.count(); }
    // Element count of the shape, or -1 when the product overflows 64 bits (never equal to a count).
    int64_t shape_size() const {
        int64_t n = 1;
        for (int32_t d : dims)
            if (__builtin_mul_overflow(n, (int64_t)d, &n)) return -1;
        return n;
    }
};

struct ParseError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

struct Reader {
    const unsigned char* p;
    const unsigned char* end;
    bool done() const { return p >= end; }
    uint64_t varint() {
        uint64_t v = 0;
        for (int shift = 0; shift < 64; shift += 7) {
            if (p >= end) throw ParseError("truncated varint");
            const unsigned char b = *p++;
            v |= (uint64_t)(b & 0x7F) << shift;
            if (!(b & 0x80)) return v;
        }
        throw ParseError("varint longer than 10 bytes");
    }
    const unsigned char* take(uint64_t n) {
        if (n > (uint64_t)(end - p)) throw ParseError("length past the end of the message");
        const unsigned char* q = p;
        p += n;
        return q;
    }
    Reader sub() {
        const uint64_t n = varint();
        const unsigned char* q = take(n);
        return Reader{q, q + n};
    }
    void skip(int wire) {
        switch (wire) {
            case 0: varint(); break;
            case 1: take(8); break;
            case 2: take(varint()); break;
            case 5: take(4); break;
            default: throw ParseError("unsupported wire type " + std::to_string(wire));
        }
    }
};

template <typename T>
T load_le(const unsigned char* q) {
    T v;
    std::memcpy(&v, q, sizeof(T));  // the wire is little-endian, as is the host
    return v;
}

void parse_policy(Reader r, Tensor& t) {
    while (!r.done()) {
        const uint64_t key = r.varint();
        const int field = (int)(key >> 3), wire = (int)(key & 7);
        if (field == 1 && wire == 2) {
            Reader q = r.sub();
            while (!q.done()) t.dims.push_back((int32_t)(uint32_t)q.varint());
        } else if (field == 1 && wire == 0) {
            t.dims.push_back((int32_t)(uint32_t)r.varint());
        } else if (field == 2 && wire == 0) {
            t.axis = (int32_t)(uint32_t)r.varint();
        } else {
            r.skip(wire);
        }
    }
}

void parse_data(Reader r, Tensor& t) {
    while (!r.done()) {
        const uint64_t key = r.varint();
        const int field = (int)(key >> 3), wire = (int)(key & 7);
        if (field == 1 && wire == 2) {
            parse_policy(r.sub(), t);
        } else if (field == 2 && wire == 2) {
            const uint64_t n = r.varint();
            if (n % 8) throw ParseError("packed double run of " + std::to_string(n) + " bytes");
            t.f64.runs.emplace_back(r.take(n), (int64_t)(n / 8));
        } else if (field == 2 && wire == 1) {
            t.f64.own.push_back(load_le<double>(r.take(8)));
        } else if (field == 3 && wire == 2) {
            const uint64_t n = r.varint();
            if (n % 4) throw ParseError("packed float run of " + std::to_string(n) + " bytes");
            t.f32.runs.emplace_back(r.take(n), (int64_t)(n / 4));
        } else if (field == 3 && wire == 5) {
            t.f32.own.push_back(load_le<float>(r.take(4)));
        } else {
            r.skip(wire);
        }
    }
}

}  // namespace

struct ar_state_dict {
    std::vector<std::unique_ptr<Mapping>> maps;
    std::map<std::string, Tensor> tensors;  // byte order of keys
    int files_loaded = 0, files_failed = 0;
};

namespace {

// One CollectionLibraryData file, in the reference's two phases: the whole message is parsed
// first (CollectionLibraryData.parseFrom: a malformed file yields nothing), then the entries are
// decoded and stored in order, and an entry that cannot be decoded stops the file with the
// entries before it kept (the per-file try/catch around the loop).
void parse_library(ar_state_dict* sd, Reader r) {
    std::vector<std::pair<std::string, Tensor>> entries;
    while (!r.done()) {
        const uint64_t key = r.varint();
        const int field = (int)(key >> 3), wire = (int)(key & 7);
        if (!(field == 1 && wire == 2)) {
            r.skip(wire);
            continue;
        }
        Reader e = r.sub();
        entries.emplace_back();
        std::string& name = entries.back().first;
        Tensor& t = entries.back().second;
        while (!e.done()) {
            const uint64_t k2 = e.varint();
            const int f2 = (int)(k2 >> 3), w2 = (int)(k2 & 7);
            if (f2 == 1 && w2 == 2) {
                Reader s = e.sub();
                name.assign((const char*)s.p, (size_t)(s.end - s.p));
            } else if (f2 == 2 && w2 == 2) {
                parse_data(e.sub(), t);
            } else {
                e.skip(w2);
            }
        }
    }
    for (auto& kv : entries) {
        const std::string& name = kv.first;
        Tensor& t = kv.second;
        if (t.dims.empty()) continue;  // CollectionEncoder.decode: no dimensions -> null, not stored
        for (int32_t d : t.dims)
            if (d <= 0) throw ParseError("entry '" + name + "': dimension " + std::to_string(d));
        if (t.count() != t.shape_size())
            throw ParseError("entry '" + name + "': " + std::to_string(t.count()) + " values for a shape of " +
                             std::to_string(t.shape_size()));
        sd->tensors[name] = std::move(t);
    }
}

int load_file(ar_state_dict* sd, const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
        ar_set_error("cannot open '%s': %s", path.c_str(), strerror(errno));
        return AR_HIP_ERR_NOT_FOUND;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        ar_set_error("cannot stat '%s': %s", path.c_str(), strerror(errno));
        return AR_HIP_ERR_NOT_FOUND;
    }
    auto m = std::make_unique<Mapping>();
    m->size = (size_t)st.st_size;
    if (m->size) {
        m->base = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m->base == MAP_FAILED) {
            m->base = nullptr;
            ::close(fd);
            ar_set_error("cannot map '%s': %s", path.c_str(), strerror(errno));
            return AR_HIP_ERR_NOT_FOUND;
        }
    }
    ::close(fd);
    const unsigned char* b = (const unsigned char*)m->base;
    sd->maps.push_back(std::move(m));
    try {
        parse_library(sd, Reader{b, b + sd->maps.back()->size});
        sd->files_loaded++;
    } catch (const ParseError& e) {
        std::fprintf(stderr, "[ar_state_dict] Error reading weights from file %s: %s\n", path.c_str(), e.what());
        sd->files_failed++;
    }
    return AR_HIP_OK;
}

template <typename Dst, typename Src>
void copy_values(const Values<Src>& v, Dst* out) {
    for (auto& r : v.runs) {
        if (sizeof(Dst) == sizeof(Src) && std::is_same<Dst, Src>::value) {
            std::memcpy(out, r.first, (size_t)r.second * sizeof(Src));
            out += r.second;
        } else {
            for (int64_t i = 0; i < r.second; i++) *out++ = (Dst)load_le<Src>(r.first + i * sizeof(Src));
        }
    }
    for (Src s : v.own) *out++ = (Dst)s;
}

const Tensor* find(const ar_state_dict* sd, const char* key) {
    auto it = sd->tensors.find(key);
    if (it == sd->tensors.end()) {
        ar_set_error("no tensor '%s' in the state dictionary", key);
        return nullptr;
    }
    return &it->second;
}

// ---- writer ------------------------------------------------------------------------------------
size_t varint_size(uint64_t v) {
    size_t n = 1;
    while (v >= 0x80) {
        v >>= 7;
        n++;
    }
    return n;
}

struct Out {
    FILE* f;
    void bytes(const void* p, size_t n) {
        if (n && std::fwrite(p, 1, n, f) != n) throw std::runtime_error(strerror(errno));
    }
    void varint(uint64_t v) {
        unsigned char b[10];
        size_t n = 0;
        while (v >= 0x80) {
            b[n++] = (unsigned char)(v | 0x80);
            v >>= 7;
        }
        b[n++] = (unsigned char)v;
        bytes(b, n);
    }
    void key(int field, int wire) { varint((uint64_t)(field << 3 | wire)); }
};

// int32 fields are encoded as sign-extended 64-bit varints (protobuf's int32 rule).
uint64_t int32_wire(int32_t v) { return (uint64_t)(int64_t)v; }

size_t policy_size(const Tensor& t) {
    size_t dims = 0;
    for (int32_t d : t.dims) dims += varint_size(int32_wire(d));
    size_t n = dims ? 1 + varint_size(dims) + dims : 0;
    if (t.axis != 0) n += 1 + varint_size(int32_wire(t.axis));  // proto3 omits a zero scalar
    return n;
}

size_t data_size(const Tensor& t, int precision) {
    const size_t ps = policy_size(t);
    size_t n = 1 + varint_size(ps) + ps;  // the policy message is always set (CollectionEncoder.encode)
    const size_t payload = (size_t)t.count() * (precision == AR_DTYPE_F64 ? 8 : 4);
    if (payload) n += 1 + varint_size(payload) + payload;
    return n;
}

// Values go out in chunks converted to the wire type; fp32 runs that are written as fp32 are
// copied as they are.
template <typename W, typename S>
void write_values(Out& o, const Values<S>& v) {
    constexpr int64_t kChunk = 1 << 16;
    std::vector<W> buf;
    auto emit = [&](const S* src_or_null, const unsigned char* raw, int64_t n) {
        for (int64_t i0 = 0; i0 < n; i0 += kChunk) {
            const int64_t len = std::min(kChunk, n - i0);
            buf.resize((size_t)len);
            for (int64_t i = 0; i < len; i++)
                buf[i] = (W)(src_or_null ? src_or_null[i0 + i] : load_le<S>(raw + (i0 + i) * sizeof(S)));
            o.bytes(buf.data(), (size_t)len * sizeof(W));
        }
    };
    for (auto& r : v.runs) {
        if (std::is_same<W, S>::value)
            o.bytes(r.first, (size_t)r.second * sizeof(S));
        else
            emit(nullptr, r.first, r.second);
    }
    emit(v.own.data(), nullptr, (int64_t)v.own.size());
}

void write_tensor_values(Out& o, const Tensor& t, int precision) {
    const int64_t n = t.count();
    if (!n) return;
    o.key(precision == AR_DTYPE_F64 ? 2 : 3, 2);
    o.varint((uint64_t)n * (precision == AR_DTYPE_F64 ? 8 : 4));
    if (precision == AR_DTYPE_F64) {
        if (t.has_f64())
            write_values<double, double>(o, t.f64);
        else
            write_values<double, float>(o, t.f32);
    } else {
        if (t.has_f64())
            write_values<float, double>(o, t.f64);
        else
            write_values<float, float>(o, t.f32);
    }
}

}  // namespace

extern "C" int ar_hip_state_dict_create(ar_state_dict** out) {
    if (!out) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *out = new ar_state_dict();
    return AR_HIP_OK;
}

extern "C" int ar_hip_state_dict_open(const char* path, ar_state_dict** out) {
    if (!path || !out) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *out = nullptr;
    struct stat st;
    if (stat(path, &st) != 0) {
        ar_set_error("weights path '%s' not found: %s", path, strerror(errno));
        return AR_HIP_ERR_NOT_FOUND;
    }
    std::vector<std::string> files;
    if (S_ISDIR(st.st_mode)) {
        DIR* d = opendir(path);
        if (!d) {
            ar_set_error("cannot list '%s': %s", path, strerror(errno));
            return AR_HIP_ERR_NOT_FOUND;
        }
        while (dirent* e = readdir(d)) {
            if (e->d_name[0] == '.') continue;  // also skips "." and ".."
            const std::string f = std::string(path) + "/" + e->d_name;
            struct stat fs;
            if (stat(f.c_str(), &fs) == 0 && S_ISREG(fs.st_mode)) files.push_back(f);
        }
        closedir(d);
        std::sort(files.begin(), files.end());
    } else {
        files.push_back(path);
    }
    auto sd = std::make_unique<ar_state_dict>();
    for (const auto& f : files) {
        const int rc = load_file(sd.get(), f);
        if (rc != AR_HIP_OK) return rc;
    }
    *out = sd.release();
    return AR_HIP_OK;
}

extern "C" int ar_hip_state_dict_destroy(ar_state_dict* sd) {
    delete sd;
    return AR_HIP_OK;
}

extern "C" int ar_hip_state_dict_size(const ar_state_dict* sd, int* count) {
    if (!sd || !count) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *count = (int)sd->tensors.size();
    return AR_HIP_OK;
}

extern "C" int ar_hip_state_dict_key(const ar_state_dict* sd, int index, const char** key) {
    if (!sd || !key) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    if (index < 0 || index >= (int)sd->tensors.size()) {
        ar_set_error("key index %d outside 0..%d", index, (int)sd->tensors.size() - 1);
        return AR_HIP_ERR_INVALID;
    }
    auto it = sd->tensors.begin();
    std::advance(it, index);
    *key = it->first.c_str();
    return AR_HIP_OK;
}

extern "C" int ar_hip_state_dict_contains(const ar_state_dict* sd, const char* key, int* found) {
    if (!sd || !key || !found) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *found = sd->tensors.count(key) ? 1 : 0;
    return AR_HIP_OK;
}

extern "C" int ar_hip_state_dict_files(const ar_state_dict* sd, int* loaded, int* failed) {
    if (!sd || !loaded || !failed) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *loaded = sd->files_loaded;
    *failed = sd->files_failed;
    return AR_HIP_OK;
}

extern "C" int ar_hip_state_dict_info(const ar_state_dict* sd, const char* key, int* ndims, int32_t* dims,
                                      int* traversal_axis, int* stored_dtype, int64_t* count) {
    if (!sd || !key || !ndims || !dims || !traversal_axis || !stored_dtype || !count) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    const Tensor* t = find(sd, key);
    if (!t) return AR_HIP_ERR_NOT_FOUND;
    if (t->dims.size() > AR_SD_MAX_DIMS) {
        ar_set_error("tensor '%s' has %d dimensions (at most %d)", key, (int)t->dims.size(), AR_SD_MAX_DIMS);
        return AR_HIP_ERR_INVALID;
    }
    *ndims = (int)t->dims.size();
    std::copy(t->dims.begin(), t->dims.end(), dims);
    *traversal_axis = t->axis;
    *stored_dtype = t->has_f64() ? AR_DTYPE_F64 : AR_DTYPE_F32;
    *count = t->count();
    return AR_HIP_OK;
}

extern "C" int ar_hip_state_dict_read(const ar_state_dict* sd, const char* key, int dtype, void* out, int64_t count) {
    if (!sd || !key || !out) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    const Tensor* t = find(sd, key);
    if (!t) return AR_HIP_ERR_NOT_FOUND;
    if (count != t->count()) {
        ar_set_error("tensor '%s': %lld values asked for, %lld stored", key, (long long)count, (long long)t->count());
        return AR_HIP_ERR_INVALID;
    }
    if (dtype == AR_DTYPE_F32) {
        if (t->has_f64())
            copy_values<float, double>(t->f64, (float*)out);
        else
            copy_values<float, float>(t->f32, (float*)out);
    } else if (dtype == AR_DTYPE_F64) {
        if (t->has_f64())
            copy_values<double, double>(t->f64, (double*)out);
        else
            copy_values<double, float>(t->f32, (double*)out);
    } else {
        ar_set_error("state dictionary values are read as fp32 or fp64, not dtype %d", dtype);
        return AR_HIP_ERR_INVALID;
    }
    return AR_HIP_OK;
}

extern "C" int ar_hip_state_dict_put(ar_state_dict* sd, const char* key, const int32_t* dims, int ndims,
                                     int traversal_axis, const void* data, int dtype, int64_t count) {
    if (!sd || !key || !dims || (!data && count)) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    if (ndims < 1 || ndims > AR_SD_MAX_DIMS) {
        ar_set_error("tensor '%s': %d dimensions (1..%d)", key, ndims, AR_SD_MAX_DIMS);
        return AR_HIP_ERR_INVALID;
    }
    Tensor t;
    t.dims.assign(dims, dims + ndims);
    t.axis = traversal_axis;
    for (int32_t d : t.dims) {
        if (d <= 0) {
            ar_set_error("tensor '%s': dimension %d", key, d);
            return AR_HIP_ERR_INVALID;
        }
    }
    if (t.shape_size() != count) {
        ar_set_error("tensor '%s': %lld values for a shape of %lld", key, (long long)count, (long long)t.shape_size());
        return AR_HIP_ERR_INVALID;
    }
    if (dtype == AR_DTYPE_F32) {
        t.f32.own.assign((const float*)data, (const float*)data + count);
    } else if (dtype == AR_DTYPE_F64) {
        t.f64.own.assign((const double*)data, (const double*)data + count);
    } else {
        ar_set_error("tensor '%s': values must be fp32 or fp64, not dtype %d", key, dtype);
        return AR_HIP_ERR_INVALID;
    }
    sd->tensors[key] = std::move(t);
    return AR_HIP_OK;
}

extern "C" int ar_hip_state_dict_save(const ar_state_dict* sd, const char* path, int precision) {
    if (!sd || !path) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    if (precision != AR_DTYPE_F32 && precision != AR_DTYPE_F64) {
        ar_set_error("save precision must be fp32 (data_32) or fp64 (data), not dtype %d", precision);
        return AR_HIP_ERR_INVALID;
    }
    FILE* f = std::fopen(path, "wb");
    if (!f) {
        ar_set_error("cannot create '%s': %s", path, strerror(errno));
        return AR_HIP_ERR_NOT_FOUND;
    }
    Out o{f};
    try {
        for (const auto& kv : sd->tensors) {
            const Tensor& t = kv.second;
            const size_t ds = data_size(t, precision);
            const size_t ks = kv.first.size();
            const size_t es = (ks ? 1 + varint_size(ks) + ks : 0) + 1 + varint_size(ds) + ds;
            o.key(1, 2);
            o.varint(es);
            if (ks) {
                o.key(1, 2);
                o.varint(ks);
                o.bytes(kv.first.data(), ks);
            }
            o.key(2, 2);
            o.varint(ds);
            const size_t ps = policy_size(t);
            o.key(1, 2);
            o.varint(ps);
            size_t dims = 0;
            for (int32_t d : t.dims) dims += varint_size(int32_wire(d));
            if (dims) {
                o.key(1, 2);
                o.varint(dims);
                for (int32_t d : t.dims) o.varint(int32_wire(d));
            }
            if (t.axis != 0) {
                o.key(2, 0);
                o.varint(int32_wire(t.axis));
            }
            write_tensor_values(o, t, precision);
        }
    } catch (const std::exception& e) {
        std::fclose(f);
        ar_set_error("writing '%s' failed: %s", path, e.what());
        return AR_HIP_ERR_INVALID;
    }
    if (std::fclose(f) != 0) {
        ar_set_error("closing '%s' failed: %s", path, strerror(errno));
        return AR_HIP_ERR_INVALID;
    }
    return AR_HIP_OK;
}

// ---- Qwen3 on top of the dictionary ---------------------------------------------------------------

extern "C" int ar_hip_qwen3_infer_config(const ar_state_dict* sd, ar_qwen3_cfg* cfg) {
    if (!sd || !cfg) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    auto get = [&](const std::string& k) -> const Tensor* {
        auto it = sd->tensors.find(k);
        return it == sd->tensors.end() ? nullptr : &it->second;
    };
    const Tensor* emb = get("model.embed_tokens.weight");
    if (!emb || emb->dims.size() != 2) {
        ar_set_error("Cannot find model.embed_tokens.weight in StateDictionary");
        return AR_HIP_ERR_INVALID;
    }
    int layers = 0;
    while (get("model.layers." + std::to_string(layers) + ".input_layernorm.weight")) layers++;
    const Tensor* qn = get("model.layers.0.self_attn.q_norm.weight");
    const Tensor* kn = get("model.layers.0.self_attn.k_norm.weight");
    if (!qn || !kn) {
        ar_set_error("Cannot find QK-Norm weights");
        return AR_HIP_ERR_INVALID;
    }
    const Tensor* w1 = get("model.layers.0.mlp.gate_proj.weight");
    if (!w1) {
        ar_set_error("Cannot find model.layers.0.mlp.gate_proj.weight in StateDictionary");
        return AR_HIP_ERR_INVALID;
    }
    ar_qwen3_cfg c;
    std::memset(&c, 0, sizeof(c));
    c.vocab_size = emb->dims[0];
    c.dim = emb->dims[1];
    c.layer_count = layers;
    c.head_count = qn->dims[0];
    c.kv_head_count = kn->dims[0];
    c.hidden_dim = w1->dims[0];
    c.seq_len = 131072;
    c.shared_weights = get("lm_head.weight") ? 0 : 1;
    c.rope_theta = 1000000.0;
    c.epsilon = 1e-6;
    c.max_batch = 1;
    c.weight_dtype = AR_DTYPE_F32;
    c.kv_dtype = AR_DTYPE_F32;
    c.qk_norm_mode = AR_QK_NORM_WHOLE;
    // (heads, head_size) gains give the head size; otherwise dim / heads (TransformerConfig.java:79)
    c.head_size = qn->dims.size() >= 2 ? qn->dims[1] : (c.head_count > 0 ? c.dim / c.head_count : 0);
    const Tensor* bq = get("model.layers.0.self_attn.q_proj.bias");
    c.qkv_bias = bq ? 1 : 0;
    *cfg = c;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_load_state_dict(ar_qwen3* m, const ar_state_dict* sd) {
    if (!m || !sd) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    std::vector<float> tmp;
    for (const auto& kv : sd->tensors) {
        const Tensor& t = kv.second;
        const void* src;
        if (!t.has_f64() && t.f32.runs.size() == 1 && t.f32.own.empty()) {
            src = t.f32.runs[0].first;  // straight from the mapped file
        } else {
            tmp.resize((size_t)t.count());
            if (t.has_f64())
                copy_values<float, double>(t.f64, tmp.data());
            else
                copy_values<float, float>(t.f32, tmp.data());
            src = tmp.data();
        }
        const int rc = ar_hip_qwen3_set_weight(m, kv.first.c_str(), src, AR_DTYPE_F32, t.count());
        if (rc == AR_HIP_ERR_NOT_FOUND) continue;  // a tensor the model has no slot for
        if (rc != AR_HIP_OK) return rc;
    }
    ar_set_error("%s", "");
    return AR_HIP_OK;
}
