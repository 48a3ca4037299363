// gguf.cpp -- GGUF v2/v3 files without ggml: the part of GgufModel / load_gguf
// (src/gguf_model.h:241-414) the MusicGen LM needs, LmConfig::from (src/mg/lm.h:60-90), and the
// adapter files of load_lora / load_mg_lora (src/ac/lora.h:113-210).
//
// The file is memory-mapped read-only; tensor data pointers point into the mapping, so
// mgx_model_create uploads straight from the page cache. Every length, count and tensor extent
// is checked against the file size before it is used.
#include "mgx.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

// shared with runtime.cpp (library-internal): the status/message convention, and the
// (in, out) of a model's projection by its GGUF name
__attribute__((visibility("hidden"))) int mgx_internal_set_error(int code, const char* msg);
__attribute__((visibility("hidden"))) bool mgx_internal_proj_shape(const mgx_model* m, const char* name, int64_t* in,
                                                                    int64_t* out);

namespace {

struct GgufError : std::runtime_error {
    int code;
    GgufError(const std::string& m, int c = MGX_ERR_INVALID) : std::runtime_error(m), code(c) {}
};

// GGUF value types (the file format's own numbering)
enum {
    G_U8 = 0, G_I8 = 1, G_U16 = 2, G_I16 = 3, G_U32 = 4, G_I32 = 5, G_F32 = 6, G_BOOL = 7, G_STR = 8,
    G_ARR = 9, G_U64 = 10, G_I64 = 11, G_F64 = 12
};

size_t scalar_size(uint32_t t) {
    switch (t) {
    case G_U8: case G_I8: case G_BOOL: return 1;
    case G_U16: case G_I16: return 2;
    case G_U32: case G_I32: case G_F32: return 4;
    case G_U64: case G_I64: case G_F64: return 8;
    }
    return 0;
}

// ggml block layouts: (bytes per block, elements per block) for the types a MusicGen LM file
// can hold (convert_musicgen_lm.py writes F16/F32, ac-quantize writes Q8_0/Q4_0).
bool type_layout(uint32_t t, size_t* bytes, int64_t* elems) {
    switch (t) {
    case 0: *bytes = 4; *elems = 1; return true;    // F32
    case 1: *bytes = 2; *elems = 1; return true;    // F16
    case 2: *bytes = 18; *elems = 32; return true;  // Q4_0
    case 3: *bytes = 20; *elems = 32; return true;  // Q4_1
    case 6: *bytes = 22; *elems = 32; return true;  // Q5_0
    case 7: *bytes = 24; *elems = 32; return true;  // Q5_1
    case 8: *bytes = 34; *elems = 32; return true;  // Q8_0
    case 30: *bytes = 2; *elems = 1; return true;   // BF16
    }
    return false;
}

struct Value {
    uint32_t type = 0;      // G_*
    uint32_t arr_type = 0;  // for G_ARR
    uint64_t count = 0;     // for G_ARR
    const uint8_t* data = nullptr;   // scalar bytes, string bytes, or the array's first element
    uint64_t len = 0;       // string length
};

struct TensorInfo {
    std::string name;
    uint32_t type = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint32_t n_dims = 0;
    uint64_t offset = 0;    // absolute, in the file
    uint64_t nbytes = 0;
};

}  // namespace

struct mgx_gguf {
    std::string path;
    const uint8_t* base = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    std::map<std::string, Value> kv;
    std::vector<TensorInfo> tensors;
    std::map<std::string, size_t> by_name;
    std::vector<std::string> adapter_names;   // targets handed out by mgx_model_set_adapters_from_gguf
    ~mgx_gguf() {
        if (base) munmap((void*)base, size);
    }
};

namespace {

struct Cursor {
    const mgx_gguf* g;
    size_t pos = 0;
    void need(uint64_t n) const {
        if (n > g->size || pos > g->size - n)
            throw GgufError("failed to open " + g->path + ": the header runs past the end of the file");
    }
    template <typename T> T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, g->base + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        need(n);
        std::string s((const char*)g->base + pos, (size_t)n);
        pos += n;
        return s;
    }
    Value value(uint32_t type, int depth = 0) {
        Value v;
        v.type = type;
        if (type == G_STR) {
            v.len = get<uint64_t>();
            need(v.len);
            v.data = g->base + pos;
            pos += v.len;
        } else if (type == G_ARR) {
            if (depth > 0) throw GgufError("failed to open " + g->path + ": nested arrays are not supported");
            v.arr_type = get<uint32_t>();
            v.count = get<uint64_t>();
            v.data = g->base + pos;
            if (v.arr_type == G_STR) {
                for (uint64_t i = 0; i < v.count; ++i) (void)str();
            } else {
                const size_t es = scalar_size(v.arr_type);
                if (!es) throw GgufError("failed to open " + g->path + ": bad array element type");
                if (v.count > (g->size - pos) / es) need(g->size + 1);
                pos += (size_t)(v.count * es);
            }
        } else {
            const size_t es = scalar_size(type);
            if (!es) throw GgufError("failed to open " + g->path + ": bad value type " + std::to_string(type));
            need(es);
            v.data = g->base + pos;
            pos += es;
        }
        return v;
    }
};

void parse(mgx_gguf* g) {
    Cursor c{g};
    if (g->size < 4 || std::memcmp(g->base, "GGUF", 4) != 0)
        throw GgufError("failed to open " + g->path + ": not a GGUF file");
    c.pos = 4;
    g->version = c.get<uint32_t>();
    if (g->version != 2 && g->version != 3)
        throw GgufError("failed to open " + g->path + ": unsupported GGUF version " + std::to_string(g->version));
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    // a tensor info takes at least 32 bytes, a key/value at least 13
    if (n_tensors > g->size / 32 || n_kv > g->size / 13)
        throw GgufError("failed to open " + g->path + ": implausible tensor or key count");
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = c.str();
        const uint32_t type = c.get<uint32_t>();
        Value v = c.value(type);
        if (g->kv.count(key)) throw GgufError("failed to open " + g->path + ": duplicate key " + key);
        g->kv.emplace(std::move(key), v);
    }
    uint64_t align = 32;
    auto al = g->kv.find("general.alignment");
    if (al != g->kv.end()) {
        if (al->second.type != G_U32) throw GgufError("failed to open " + g->path + ": general.alignment is not u32");
        uint32_t a;
        std::memcpy(&a, al->second.data, 4);
        if (a == 0 || (a & (a - 1))) throw GgufError("failed to open " + g->path + ": bad alignment");
        align = a;
    }
    std::vector<TensorInfo> ts((size_t)n_tensors);
    for (TensorInfo& t : ts) {
        t.name = c.str();
        t.n_dims = c.get<uint32_t>();
        if (t.n_dims < 1 || t.n_dims > 4)
            throw GgufError("failed to open " + g->path + ": tensor " + t.name + " has " + std::to_string(t.n_dims) + " dims");
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            t.ne[d] = c.get<int64_t>();
            if (t.ne[d] < 0) throw GgufError("failed to open " + g->path + ": negative dim in " + t.name);
        }
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        size_t bb;
        int64_t be;
        if (!type_layout(t.type, &bb, &be))
            throw GgufError("failed to open " + g->path + ": tensor " + t.name + " has an unsupported type " +
                            std::to_string(t.type));
        if (t.ne[0] % be) throw GgufError("failed to open " + g->path + ": rows of " + t.name + " split a block");
        uint64_t rows = 1;
        for (int d = 1; d < 4; ++d) {
            if (t.ne[d] && rows > UINT64_MAX / (uint64_t)t.ne[d]) throw GgufError("failed to open " + g->path + ": tensor too large");
            rows *= (uint64_t)t.ne[d];
        }
        const uint64_t row_bytes = (uint64_t)(t.ne[0] / be) * bb;
        if (rows && row_bytes > UINT64_MAX / rows) throw GgufError("failed to open " + g->path + ": tensor too large");
        t.nbytes = row_bytes * rows;
        if (g->by_name.count(t.name)) throw GgufError("failed to open " + g->path + ": duplicate tensor " + t.name);
        g->by_name[t.name] = (size_t)(&t - ts.data());
    }
    const uint64_t data_off = (c.pos + align - 1) / align * align;
    for (TensorInfo& t : ts) {
        if (t.offset % align) throw GgufError("failed to open " + g->path + ": misaligned tensor " + t.name);
        const uint64_t off = data_off + t.offset;
        // the short-read check of load_gguf (gguf_model.h:384-389)
        if (off > g->size || t.nbytes > g->size - off) {
            const uint64_t avail = off < g->size ? g->size - off : 0;
            throw GgufError("short read while loading tensor " + t.name + " from " + g->path + ": needed " +
                            std::to_string(t.nbytes) + " bytes at offset " + std::to_string(off) + ", " +
                            std::to_string(avail < t.nbytes ? avail : t.nbytes) + " available (file size " +
                            std::to_string(g->size) + ")");
        }
        t.offset = off;
    }
    g->tensors = std::move(ts);
}

const Value& key(const mgx_gguf* g, const std::string& k) {
    auto it = g->kv.find(k);
    if (it == g->kv.end()) throw GgufError("missing key: " + k);
    return it->second;
}
uint32_t u32(const mgx_gguf* g, const std::string& k) {
    const Value& v = key(g, k);
    if (v.type != G_U32) throw GgufError("key is not u32: " + k);
    uint32_t x;
    std::memcpy(&x, v.data, 4);
    return x;
}
float f32(const mgx_gguf* g, const std::string& k) {
    const Value& v = key(g, k);
    if (v.type != G_F32) throw GgufError("key is not f32: " + k);
    float x;
    std::memcpy(&x, v.data, 4);
    return x;
}
std::string str(const mgx_gguf* g, const std::string& k) {
    const Value& v = key(g, k);
    if (v.type != G_STR) throw GgufError("key is not string: " + k);
    return std::string((const char*)v.data, (size_t)v.len);
}
bool has(const mgx_gguf* g, const std::string& k) { return g->kv.count(k) != 0; }

mgx_tensor view(const mgx_gguf* g, const TensorInfo& t) {
    mgx_tensor o{};
    o.name = t.name.c_str();
    o.type = (int32_t)t.type;
    for (int d = 0; d < 4; ++d) o.ne[d] = t.ne[d];
    o.data = g->base + t.offset;
    o.nbytes = t.nbytes;
    return o;
}
const TensorInfo* find(const mgx_gguf* g, const std::string& n) {
    auto it = g->by_name.find(n);
    return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
}

// LmConfig::from (lm.h:60-90)
mgx_lm_config lm_config(const mgx_gguf* g) {
    if (str(g, "ac.architecture") != "audiocraft") throw GgufError("not an audiocraft GGUF");
    if (u32(g, "ac.format_version") != 1) throw GgufError("unsupported audiocraft GGUF version");
    if (str(g, "ac.lm.family") != "musicgen") throw GgufError("not a MusicGen LM GGUF");
    mgx_lm_config c{};
    c.dim = (int32_t)u32(g, "ac.lm.dim");
    c.layers = (int32_t)u32(g, "ac.lm.layers");
    c.heads = (int32_t)u32(g, "ac.lm.heads");
    c.head_dim = (int32_t)u32(g, "ac.lm.head_dim");
    c.ff_dim = (int32_t)u32(g, "ac.lm.ff_dim");
    c.cond_dim = (int32_t)u32(g, "ac.lm.cond_dim");
    c.n_q = (int32_t)u32(g, "ac.lm.n_q");
    c.card = (int32_t)u32(g, "ac.lm.card");
    c.special_token_id = (int32_t)u32(g, "ac.lm.special_token_id");
    c.pos_denominator = (int32_t)u32(g, "ac.lm.pos_denominator");
    c.max_period = f32(g, "ac.lm.max_period");
    c.norm_eps = f32(g, "ac.lm.norm_eps");
    c.cfg_coef = f32(g, "ac.lm.cfg_coef");
    (void)u32(g, "ac.lm.sample_rate");     // read (and required) by LmConfig::from
    (void)f32(g, "ac.lm.max_duration");
    if (c.dim != c.heads * c.head_dim) throw GgufError("LM dim does not equal heads * head_dim");
    if (c.special_token_id != c.card) throw GgufError("special_token_id should be card: it is the extra embedding row");
    return c;
}

std::vector<int32_t> i32s(const mgx_gguf* g, const std::string& k) {
    const Value& v = key(g, k);
    if (v.type != G_ARR || v.arr_type != G_I32) throw GgufError("key is not an i32 array: " + k);
    std::vector<int32_t> out((size_t)v.count);
    if (v.count) std::memcpy(out.data(), v.data, 4 * (size_t)v.count);
    return out;
}

// SeanetConfig::from (seanet.h:60-92)
mgx_codec_config codec_config(const mgx_gguf* g) {
    if (str(g, "ac.architecture") != "audiocraft") throw GgufError("not an audiocraft GGUF");
    if (u32(g, "ac.format_version") != 1) throw GgufError("unsupported audiocraft GGUF version");
    mgx_codec_config c{};
    const std::string quantizer = str(g, "ac.codec.quantizer");
    c.elu = str(g, "ac.codec.activation") == "ELU" ? 1 : 0;
    c.channels = (int32_t)u32(g, "ac.codec.channels");
    c.n_filters = (int32_t)u32(g, "ac.codec.n_filters");
    c.n_residual_layers = (int32_t)u32(g, "ac.codec.n_residual_layers");
    c.kernel_size = (int32_t)u32(g, "ac.codec.kernel_size");
    c.residual_kernel_size = (int32_t)u32(g, "ac.codec.residual_kernel_size");
    c.last_kernel_size = (int32_t)u32(g, "ac.codec.last_kernel_size");
    c.dilation_base = (int32_t)u32(g, "ac.codec.dilation_base");
    c.compress = (int32_t)u32(g, "ac.codec.compress");
    c.lstm_layers = (int32_t)u32(g, "ac.codec.lstm_layers");
    c.latent_dim = (int32_t)u32(g, "ac.codec.latent_dim");
    (void)u32(g, "ac.codec.encoder_dim");
    c.sample_rate = (int32_t)u32(g, "ac.codec.sample_rate");
    c.hop_length = (int32_t)u32(g, "ac.codec.hop_length");
    if (quantizer == "rvq") {
        c.rvq = 1;
        c.rvq_n_q = (int32_t)u32(g, "ac.codec.rvq_n_q");
        c.rvq_bins = (int32_t)u32(g, "ac.codec.rvq_bins");
    }
    c.frame_rate = (int32_t)u32(g, "ac.codec.frame_rate");
    const std::vector<int32_t> r = i32s(g, "ac.codec.ratios");
    if (r.empty()) throw GgufError("codec has no ratios");
    if (r.size() > 8) throw GgufError("codec has more than 8 ratios");
    int hop = 1;
    for (size_t i = 0; i < r.size(); ++i) {
        c.ratios[i] = r[i];
        hop *= r[i];
    }
    c.n_ratios = (int32_t)r.size();
    if (hop != c.hop_length) throw GgufError("codec ratio product disagrees with the declared hop length");
    return c;
}

// T5EncoderConfig::from (t5.h:31-43): the ac.t5.* keys, each required
mgx_t5_config t5_config(const mgx_gguf* g) {
    mgx_t5_config c{};
    c.dim = (int32_t)u32(g, "ac.t5.dim");
    c.layers = (int32_t)u32(g, "ac.t5.layers");
    c.heads = (int32_t)u32(g, "ac.t5.heads");
    c.head_dim = (int32_t)u32(g, "ac.t5.head_dim");
    c.intermediate = (int32_t)u32(g, "ac.t5.intermediate");
    c.vocab = (int32_t)u32(g, "ac.t5.vocab");
    c.relative_buckets = (int32_t)u32(g, "ac.t5.relative_buckets");
    c.relative_max_distance = (int32_t)u32(g, "ac.t5.relative_max_distance");
    c.eps = f32(g, "ac.t5.eps");
    return c;
}

template <typename F> int guarded(F&& f) {
    try {
        f();
        return MGX_OK;
    } catch (const GgufError& e) {
        return mgx_internal_set_error(e.code, e.what());
    } catch (const std::exception& e) {
        return mgx_internal_set_error(MGX_ERR_INVALID, e.what());
    }
}

}  // namespace

extern "C" {

int mgx_gguf_open(const char* path, mgx_gguf** out) {
    return guarded([&] {
        if (!path || !out) throw GgufError("null argument");
        *out = nullptr;
        auto g = std::make_unique<mgx_gguf>();
        g->path = path;
        const int fd = open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) throw GgufError("failed to open " + g->path + ": " + std::strerror(errno));
        struct stat st {};
        if (fstat(fd, &st) != 0) {
            const int e = errno;
            close(fd);
            throw GgufError("cannot read " + g->path + ": " + std::strerror(e));
        }
        g->size = (size_t)st.st_size;
        if (g->size == 0) {
            close(fd);
            throw GgufError("failed to open " + g->path + ": empty file");
        }
        void* p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        close(fd);
        if (p == MAP_FAILED) throw GgufError("cannot read " + g->path + ": " + std::strerror(errno));
        g->base = (const uint8_t*)p;
        parse(g.get());
        *out = g.release();
    });
}

void mgx_gguf_close(mgx_gguf* g) { delete g; }

int32_t mgx_gguf_tensor_count(const mgx_gguf* g) { return g ? (int32_t)g->tensors.size() : -1; }

int mgx_gguf_tensor(const mgx_gguf* g, int32_t i, mgx_tensor* out) {
    return guarded([&] {
        if (!g || !out) throw GgufError("null argument");
        if (i < 0 || (size_t)i >= g->tensors.size()) throw GgufError("tensor index out of range");
        *out = view(g, g->tensors[(size_t)i]);
    });
}

int mgx_gguf_find_tensor(const mgx_gguf* g, const char* name, mgx_tensor* out) {
    return guarded([&] {
        if (!g || !name || !out) throw GgufError("null argument");
        const TensorInfo* t = find(g, name);
        if (!t) throw GgufError(std::string("missing tensor: ") + name);
        *out = view(g, *t);
    });
}

int mgx_gguf_u32(const mgx_gguf* g, const char* k, uint32_t* out) {
    return guarded([&] {
        if (!g || !k || !out) throw GgufError("null argument");
        *out = u32(g, k);
    });
}

int mgx_gguf_f32(const mgx_gguf* g, const char* k, float* out) {
    return guarded([&] {
        if (!g || !k || !out) throw GgufError("null argument");
        *out = f32(g, k);
    });
}

int mgx_gguf_string(const mgx_gguf* g, const char* k, char* buf, uint64_t cap, uint64_t* len) {
    return guarded([&] {
        if (!g || !k) throw GgufError("null argument");
        const std::string s = str(g, k);
        if (len) *len = s.size();
        if (buf && cap) {
            const size_t n = s.size() < cap - 1 ? s.size() : (size_t)cap - 1;
            std::memcpy(buf, s.data(), n);
            buf[n] = '\0';
        }
    });
}

int mgx_gguf_lm_config(const mgx_gguf* g, mgx_lm_config* out) {
    return guarded([&] {
        if (!g || !out) throw GgufError("null argument");
        *out = lm_config(g);
    });
}

int mgx_model_create_from_gguf(const mgx_gguf* g, mgx_model** out) {
    mgx_lm_config c{};
    std::vector<mgx_tensor> ts;
    const int rc = guarded([&] {
        if (!g || !out) throw GgufError("null argument");
        *out = nullptr;
        c = lm_config(g);
        ts.reserve(g->tensors.size());
        for (const TensorInfo& t : g->tensors) ts.push_back(view(g, t));
    });
    if (rc != MGX_OK) return rc;
    return mgx_model_create(&c, ts.data(), (int32_t)ts.size(), out);
}

int mgx_gguf_t5_config(const mgx_gguf* g, mgx_t5_config* out) {
    return guarded([&] {
        if (!g || !out) throw GgufError("null argument");
        *out = t5_config(g);
    });
}

int mgx_t5_create_from_gguf(const mgx_gguf* g, mgx_t5** out) {
    mgx_t5_config c{};
    std::vector<mgx_tensor> ts;
    const int rc = guarded([&] {
        if (!g || !out) throw GgufError("null argument");
        *out = nullptr;
        c = t5_config(g);
        ts.reserve(g->tensors.size());
        for (const TensorInfo& t : g->tensors) ts.push_back(view(g, t));
    });
    if (rc != MGX_OK) return rc;
    return mgx_t5_create(&c, ts.data(), (int32_t)ts.size(), out);
}

int mgx_gguf_codec_config(const mgx_gguf* g, mgx_codec_config* out) {
    return guarded([&] {
        if (!g || !out) throw GgufError("null argument");
        *out = codec_config(g);
    });
}

int mgx_codec_create_from_gguf(const mgx_gguf* g, mgx_codec** out) {
    mgx_codec_config c{};
    std::vector<mgx_tensor> ts;
    const int rc = guarded([&] {
        if (!g || !out) throw GgufError("null argument");
        *out = nullptr;
        c = codec_config(g);
        ts.reserve(g->tensors.size());
        for (const TensorInfo& t : g->tensors) ts.push_back(view(g, t));
    });
    if (rc != MGX_OK) return rc;
    return mgx_codec_create(&c, ts.data(), (int32_t)ts.size(), out);
}

int mgx_model_set_adapters_from_gguf(mgx_model* model, const mgx_gguf* g, const mgx_gguf* base, float strength) {
    std::vector<mgx_adapter> ads;
    const int rc = guarded([&] {
        if (!model || !g) throw GgufError("null argument");
        // load_mg_lora + load_lora (lora.h:113-176, 195-210)
        if (str(g, "general.architecture") != "ac-musicgen-lora") throw GgufError("not a MusicGen adapter");
        if (u32(g, "ac.lora.version") != 1) throw GgufError("unsupported adapter");
        const int rank = (int)u32(g, "ac.lora.rank");
        const float alpha = f32(g, "ac.lora.alpha");
        const std::string type = has(g, "ac.lora.type") ? str(g, "ac.lora.type") : "lora";
        if (type != "lora" && type != "dora-rows") throw GgufError("unsupported adapter type: " + type);
        const bool dora = type == "dora-rows";
        if (rank <= 0 || !std::isfinite(alpha) || alpha <= 0 || !std::isfinite(strength))
            throw GgufError("invalid adapter rank, alpha or strength");
        const std::string suffix = ".lora_A";
        mgx_gguf* gm = const_cast<mgx_gguf*>(g);
        gm->adapter_names.clear();
        std::vector<const TensorInfo*> as;
        for (const TensorInfo& t : g->tensors)
            if (t.name.size() > suffix.size() && t.name.compare(t.name.size() - suffix.size(), suffix.size(), suffix) == 0)
                as.push_back(&t);
        for (const TensorInfo* A : as) {
            const std::string stem = A->name.substr(0, A->name.size() - suffix.size());
            const TensorInfo* B = find(g, stem + ".lora_B");
            if (!B) throw GgufError("missing tensor: " + stem + ".lora_B");
            if (base) {
                const TensorInfo* W = find(base, stem);
                if (!W) throw GgufError("missing tensor: " + stem);
                if (W->ne[0] != A->ne[0] || W->ne[1] != B->ne[1] || W->ne[2] != 1 || W->ne[3] != 1)
                    throw GgufError("adapter shape mismatch: " + stem);
            }
            int64_t win = 0, wout = 0;
            if (!mgx_internal_proj_shape(model, stem.c_str(), &win, &wout))
                throw GgufError("unsupported MusicGen adapter target: " + stem);
            if (A->ne[0] != win || B->ne[1] != wout) throw GgufError("adapter shape mismatch: " + stem);
            if (A->type != 0 || B->type != 0 || A->ne[1] != rank || B->ne[0] != rank || A->ne[2] != 1 ||
                A->ne[3] != 1 || B->ne[2] != 1 || B->ne[3] != 1)
                throw GgufError("adapter shape mismatch: " + stem);
            const TensorInfo* M = nullptr;
            if (dora) {
                M = find(g, stem + ".magnitude");
                if (!M) throw GgufError("missing tensor: " + stem + ".magnitude");
                if (M->type != 0 || M->ne[0] != B->ne[1] || M->ne[1] != 1 || M->ne[2] != 1 || M->ne[3] != 1)
                    throw GgufError("DoRA magnitude shape mismatch: " + stem);
            }
            gm->adapter_names.push_back(stem);
            mgx_adapter a{};
            a.A = (const float*)(g->base + A->offset);
            a.B = (const float*)(g->base + B->offset);
            a.magnitude = M ? (const float*)(g->base + M->offset) : nullptr;
            a.rank = rank;
            a.alpha = alpha;
            a.strength = strength;
            ads.push_back(a);
        }
        if (ads.empty() || g->tensors.size() != (dora ? 3 : 2) * ads.size())
            throw GgufError("empty or incomplete adapter");
        if (base && has(g, "ac.lora.base_name") && has(base, "general.name") &&
            str(g, "ac.lora.base_name") != str(base, "general.name"))
            throw GgufError("adapter base model name does not match");
        for (size_t i = 0; i < ads.size(); ++i) ads[i].target = gm->adapter_names[i].c_str();
    });
    if (rc != MGX_OK) return rc;
    return mgx_model_set_adapters(model, ads.data(), (int32_t)ads.size());
}

}  // extern "C"
