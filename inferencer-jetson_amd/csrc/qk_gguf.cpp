// qk_gguf.cpp - GGUF v3 reader, tensor-table validation and device upload.
//
// Replaces the reference's Reader and GGUF structs (inferencer.cu:130-176,
// 204-340) and the model lookup of FastRunner's constructor
// (inferencer.cu:1196-1214).  The file is mapped once and parsed from the
// mapping with a bounds-checked cursor, so a truncated or corrupt header is
// a status code, never a read past the end.  What is read follows the
// reference: scalar metadata kept as doubles (string and array values
// skipped), tokenizer.ggml.tokens / merges kept as string arrays, tensor
// infos of FP32, FP16, Q4_K and Q6_K, general.alignment (default 32, a power
// of two) and the aligned data start.  Checks the reference does not make:
// offset + bytes must lie inside the data section (the reference tests only
// offset < size, inferencer.cu:282), offsets must be multiples of the
// alignment (the device kernels need 16-byte aligned tensors), element
// counts must not overflow, and tensor names must be unique.
#include "qk_internal.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

struct qk_gguf {
    int fd = -1;
    void *mapping = MAP_FAILED;
    uint64_t file_size = 0, data_start = 0, alignment = 32;
    std::unordered_map<std::string, double> params;
    std::unordered_map<std::string, std::string> strings;
    std::vector<std::string> tokens, merges;
    std::vector<std::string> names;
    std::vector<qk_gguf_tensor> tensors;
    std::unordered_map<std::string, size_t> index;
    void *device = nullptr;
};

namespace qk {
namespace {

// GGUF metadata value types (the GGUF v3 specification; the reference's
// Reader::scalar / skip, inferencer.cu:149-175).
enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};
constexpr uint64_t kMaxString = 100000000;   // inferencer.cu:142
constexpr uint64_t kMaxArray = 10000000;     // inferencer.cu:167

struct FormatError {
    std::string what;
};

class Cursor {
  public:
    Cursor(const uint8_t *base, uint64_t size) : base_(base), size_(size) {}
    uint64_t pos() const { return pos_; }
    uint64_t left() const { return size_ - pos_; }

    template <class T>
    T number() {
        need(sizeof(T), "header ends before its metadata does");
        T v;
        std::memcpy(&v, base_ + pos_, sizeof(T));
        pos_ += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = number<uint64_t>();
        if (n > kMaxString) throw FormatError{"metadata string over the 1e8-byte limit"};
        need(n, "metadata string runs past the end of the file");
        std::string s(reinterpret_cast<const char *>(base_ + pos_), n);
        pos_ += n;
        return s;
    }
    double scalar(uint32_t type) {
        switch (type) {
            case kU8: return number<uint8_t>();
            case kI8: return number<int8_t>();
            case kU16: return number<uint16_t>();
            case kI16: return number<int16_t>();
            case kU32: return number<uint32_t>();
            case kI32: return number<int32_t>();
            case kF32: return number<float>();
            case kBool: return number<uint8_t>();
            case kU64: return static_cast<double>(number<uint64_t>());
            case kI64: return static_cast<double>(number<int64_t>());
            case kF64: return number<double>();
            default: throw FormatError{"unsupported GGUF metadata type " + std::to_string(type)};
        }
    }
    void skip(uint32_t type, int depth = 0) {
        if (type == kString) {
            str();
        } else if (type == kArray) {
            if (depth > 8) throw FormatError{"GGUF arrays nested too deeply"};
            const uint32_t element = number<uint32_t>();
            const uint64_t count = number<uint64_t>();
            if (count > kMaxArray) throw FormatError{"metadata array over the 1e7-entry limit"};
            for (uint64_t i = 0; i < count; ++i) skip(element, depth + 1);
        } else {
            scalar(type);
        }
    }

  private:
    void need(uint64_t n, const char *what) const {
        if (n > size_ - pos_) throw FormatError{what};
    }
    const uint8_t *base_;
    uint64_t size_, pos_ = 0;
};

// Bytes of a tensor of `elements` values (inferencer.cu:246-259); other
// storage types are a format error, as in the reference.
uint64_t storage_bytes(uint32_t type, uint64_t elements, const std::string &name) {
    switch (type) {
        case 0: return elements * 4;
        case 1: return elements * 2;
        case QK_TYPE_Q4_K:
        case QK_TYPE_Q6_K:
            if (elements % 256) throw FormatError{"block-quantized tensor whose size is not a multiple of 256: " + name};
            return elements / 256 * (type == QK_TYPE_Q4_K ? 144 : 210);
        default: throw FormatError{"unsupported tensor storage type " + std::to_string(type) + ": " + name};
    }
}

void parse(qk_gguf &g) {
    Cursor r(static_cast<const uint8_t *>(g.mapping), g.file_size);
    const uint32_t magic = r.number<uint32_t>();
    if (std::memcmp(&magic, "GGUF", 4)) throw FormatError{"bad magic: no GGUF header"};
    const uint32_t version = r.number<uint32_t>();
    if (version != 3) throw FormatError{"GGUF version " + std::to_string(version) + " found; this reader takes version 3"};
    const uint64_t n_tensors = r.number<uint64_t>(), n_meta = r.number<uint64_t>();
    // Every entry takes at least 8 + 4 bytes of the file, which bounds both
    // counts before anything is reserved.
    if (n_tensors > g.file_size / 12 || n_meta > g.file_size / 12) throw FormatError{"invalid GGUF entry counts"};
    for (uint64_t i = 0; i < n_meta; ++i) {
        std::string key = r.str();
        const uint32_t type = r.number<uint32_t>();
        if (key == "tokenizer.ggml.tokens" || key == "tokenizer.ggml.merges") {
            if (type != kArray || r.number<uint32_t>() != kString)
                throw FormatError{"token or merge list with non-string entries: " + key};
            const uint64_t count = r.number<uint64_t>();
            // Each entry needs at least its 8-byte length, which bounds the
            // reservation by the bytes left in the file.
            if (count > kMaxArray || count > r.left() / 8)
                throw FormatError{"metadata array over the 1e7-entry limit or past the end of the file"};
            auto &target = key == "tokenizer.ggml.tokens" ? g.tokens : g.merges;
            target.clear();
            target.reserve(count);
            for (uint64_t j = 0; j < count; ++j) target.push_back(r.str());
        } else if (type == kString) {
            g.strings[key] = r.str();
        } else if (type == kArray) {
            r.skip(type);
        } else {
            g.params[key] = r.scalar(type);
        }
    }
    g.names.reserve(n_tensors);
    g.tensors.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        std::string name = r.str();
        qk_gguf_tensor t{};
        const uint32_t nd = r.number<uint32_t>();
        if (nd == 0 || nd > 4) throw FormatError{"invalid tensor dimensions: " + name};
        t.n_dims = static_cast<int>(nd);
        uint64_t elements = 1;
        for (uint32_t j = 0; j < nd; ++j) {
            const uint64_t d = r.number<uint64_t>();
            if (d == 0 || d > (uint64_t(1) << 40) || elements > (uint64_t(1) << 48) / d)
                throw FormatError{"invalid tensor dimensions: " + name};
            t.dims[j] = static_cast<int64_t>(d);
            elements *= d;
        }
        for (uint32_t j = nd; j < 4; ++j) t.dims[j] = 1;
        const uint32_t type = r.number<uint32_t>();
        t.type = static_cast<int>(type);
        t.offset = r.number<uint64_t>();
        t.bytes = storage_bytes(type, elements, name);
        if (g.index.count(name)) throw FormatError{"duplicate tensor name: " + name};
        g.index.emplace(name, g.tensors.size());
        g.names.push_back(std::move(name));
        g.tensors.push_back(t);
    }
    auto al = g.params.find("general.alignment");
    if (al != g.params.end()) {
        const double a = al->second;
        if (!(a >= 1.0 && a <= 1073741824.0) || a != static_cast<double>(static_cast<uint64_t>(a)))
            throw FormatError{"general.alignment must be a positive power of two"};
        g.alignment = static_cast<uint64_t>(a);
    }
    if (g.alignment & (g.alignment - 1)) throw FormatError{"general.alignment must be a positive power of two"};
    g.data_start = (r.pos() + g.alignment - 1) & ~(g.alignment - 1);
    if (g.file_size <= g.data_start) throw FormatError{"invalid GGUF file size: no tensor data"};
    const uint64_t data_bytes = g.file_size - g.data_start;
    const uint8_t *data = static_cast<const uint8_t *>(g.mapping) + g.data_start;
    for (size_t i = 0; i < g.tensors.size(); ++i) {
        qk_gguf_tensor &t = g.tensors[i];
        if (t.offset > data_bytes || t.bytes > data_bytes - t.offset)
            throw FormatError{"tensor data outside the file: " + g.names[i]};
        if (t.offset % g.alignment) throw FormatError{"tensor offset not aligned: " + g.names[i]};
        t.name = g.names[i].c_str();
        t.host = data + t.offset;
    }
}

void release(qk_gguf *g) {
    if (g->device) (void)hipFree(g->device);
    if (g->mapping != MAP_FAILED) munmap(g->mapping, g->file_size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

}  // namespace
}  // namespace qk

extern "C" {

int qk_gguf_open(const char *path, qk_gguf **out) {
    if (!path || !out) return qk::fail(QK_ERR_INVALID_ARG, "qk_gguf_open: null argument");
    *out = nullptr;
    qk_gguf *g = new qk_gguf;
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) {
        qk::release(g);
        return qk::fail(QK_ERR_IO, std::string("cannot open GGUF: ") + path);
    }
    struct stat st {};
    if (fstat(g->fd, &st) || st.st_size < 24) {
        qk::release(g);
        return qk::fail(QK_ERR_FORMAT, std::string("invalid GGUF file size: ") + path);
    }
    g->file_size = static_cast<uint64_t>(st.st_size);
    g->mapping = mmap(nullptr, g->file_size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (g->mapping == MAP_FAILED) {
        qk::release(g);
        return qk::fail(QK_ERR_IO, std::string("GGUF mmap failed: ") + path);
    }
    try {
        qk::parse(*g);
    } catch (const qk::FormatError &e) {
        qk::release(g);
        return qk::fail(QK_ERR_FORMAT, e.what + " (" + path + ")");
    } catch (const std::bad_alloc &) {
        qk::release(g);
        return qk::fail(QK_ERR_LIMIT, std::string("GGUF tables too large for host memory: ") + path);
    }
    *out = g;
    return qk::ok();
}

int qk_gguf_close(qk_gguf *g) {
    if (!g) return qk::fail(QK_ERR_INVALID_ARG, "qk_gguf_close: null handle");
    qk::release(g);
    return qk::ok();
}

int qk_gguf_param(const qk_gguf *g, const char *key, double *value) {
    if (!g || !key || !value) return qk::fail(QK_ERR_INVALID_ARG, "qk_gguf_param: null argument");
    auto it = g->params.find(key);
    if (it == g->params.end()) return qk::fail(QK_ERR_INVALID_ARG, std::string("no metadata key ") + key);
    *value = it->second;
    return qk::ok();
}

const char *qk_gguf_string(const qk_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->strings.find(key);
    return it == g->strings.end() ? nullptr : it->second.c_str();
}

int64_t qk_gguf_tensor_count(const qk_gguf *g) { return g ? static_cast<int64_t>(g->tensors.size()) : -1; }

int qk_gguf_tensor_at(const qk_gguf *g, int64_t i, qk_gguf_tensor *out) {
    if (!g || !out || i < 0 || i >= static_cast<int64_t>(g->tensors.size()))
        return qk::fail(QK_ERR_INVALID_ARG, "qk_gguf_tensor_at: null argument or index out of range");
    *out = g->tensors[static_cast<size_t>(i)];
    return qk::ok();
}

int qk_gguf_find_tensor(const qk_gguf *g, const char *name, qk_gguf_tensor *out) {
    if (!g || !name || !out) return qk::fail(QK_ERR_INVALID_ARG, "qk_gguf_find_tensor: null argument");
    auto it = g->index.find(name);
    if (it == g->index.end()) return qk::fail(QK_ERR_INVALID_ARG, std::string("no tensor named ") + name);
    *out = g->tensors[it->second];
    return qk::ok();
}

int64_t qk_gguf_token_count(const qk_gguf *g, int which) {
    if (!g || (which != 0 && which != 1)) return -1;
    return static_cast<int64_t>((which ? g->merges : g->tokens).size());
}

const char *qk_gguf_token(const qk_gguf *g, int which, int64_t i, int64_t *length) {
    if (!g || (which != 0 && which != 1)) return nullptr;
    const auto &v = which ? g->merges : g->tokens;
    if (i < 0 || i >= static_cast<int64_t>(v.size())) return nullptr;
    if (length) *length = static_cast<int64_t>(v[static_cast<size_t>(i)].size());
    return v[static_cast<size_t>(i)].data();
}

int qk_gguf_data(const qk_gguf *g, const void **host, uint64_t *bytes, uint64_t *alignment) {
    if (!g) return qk::fail(QK_ERR_INVALID_ARG, "qk_gguf_data: null handle");
    if (host) *host = static_cast<const uint8_t *>(g->mapping) + g->data_start;
    if (bytes) *bytes = g->file_size - g->data_start;
    if (alignment) *alignment = g->alignment;
    return qk::ok();
}

int qk_gguf_upload(qk_gguf *g, qk_stream stream) {
    if (!g) return qk::fail(QK_ERR_INVALID_ARG, "qk_gguf_upload: null handle");
    if (g->device) return qk::ok();
    const uint64_t bytes = g->file_size - g->data_start;
    size_t free_bytes = 0, total_bytes = 0;
    if (hipMemGetInfo(&free_bytes, &total_bytes) != hipSuccess)
        return qk::fail(QK_ERR_DEVICE, "qk_gguf_upload: device memory query failed");
    if (free_bytes < bytes + (64u << 20))    // inferencer.cu:331-333
        return qk::fail(QK_ERR_LIMIT, "qk_gguf_upload: not enough free device memory for the weights");
    if (hipMalloc(&g->device, bytes) != hipSuccess) {
        g->device = nullptr;
        return qk::fail(QK_ERR_DEVICE, "qk_gguf_upload: device allocation failed");
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (hipMemcpyAsync(g->device, static_cast<const uint8_t *>(g->mapping) + g->data_start, bytes,
                       hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        (void)hipFree(g->device);
        g->device = nullptr;
        return qk::fail(QK_ERR_DEVICE, "qk_gguf_upload: weight upload failed");
    }
    for (qk_gguf_tensor &t : g->tensors) t.device = static_cast<const uint8_t *>(g->device) + t.offset;
    return qk::ok();
}

// FastRunner's model lookup (inferencer.cu:1196-1214) for any Llama shape the
// drivers support: the llama.* hyper-parameters, then every tensor by its
// GGUF name with its storage type and dimensions checked.
int qk_gguf_llama(const qk_gguf *g, int context, qk_llama_config *cfg, qk_llama_weights *w,
                  qk_llama_layer *layers, int max_layers) {
    if (!g || !cfg || !w || !layers) return qk::fail(QK_ERR_INVALID_ARG, "qk_gguf_llama: null argument");
    if (!g->device) return qk::fail(QK_ERR_INVALID_ARG, "qk_gguf_llama: call qk_gguf_upload first");
    if (context < 1) return qk::fail(QK_ERR_INVALID_ARG, "qk_gguf_llama: context must be positive");
    auto param = [&](const char *key, double &v) { return qk_gguf_param(g, key, &v); };
    double dim, layers_d, heads, kv_heads, hidden, eps, theta;
    int st;
    if ((st = param("llama.embedding_length", dim)) || (st = param("llama.block_count", layers_d)) ||
        (st = param("llama.attention.head_count", heads)) || (st = param("llama.attention.head_count_kv", kv_heads)) ||
        (st = param("llama.feed_forward_length", hidden)) ||
        (st = param("llama.attention.layer_norm_rms_epsilon", eps)) || (st = param("llama.rope.freq_base", theta)))
        return st;
    qk_gguf_tensor embd{};
    if ((st = qk_gguf_find_tensor(g, "token_embd.weight", &embd))) return st;
    double vocab = static_cast<double>(embd.dims[1]);
    auto vit = g->params.find("llama.vocab_size");
    if (vit != g->params.end()) vocab = vit->second;
    auto as_int = [](double v) { return v >= 1.0 && v <= 1e9 && v == static_cast<double>(static_cast<int>(v)); };
    if (!as_int(dim) || !as_int(layers_d) || !as_int(heads) || !as_int(kv_heads) || !as_int(hidden) || !as_int(vocab))
        return qk::fail(QK_ERR_SHAPE, "qk_gguf_llama: invalid llama hyper-parameters");
    qk_llama_config c{};
    c.dim = static_cast<int>(dim);
    c.layers = static_cast<int>(layers_d);
    c.heads = static_cast<int>(heads);
    c.kv_heads = static_cast<int>(kv_heads);
    c.hidden = static_cast<int>(hidden);
    c.vocab = static_cast<int>(vocab);
    c.context = context;
    c.eps = static_cast<float>(eps);
    c.rope_theta = static_cast<float>(theta);
    if (c.dim % c.heads || c.heads % c.kv_heads)
        return qk::fail(QK_ERR_SHAPE, "qk_gguf_llama: heads do not divide the embedding");
    if (c.layers > max_layers) return qk::fail(QK_ERR_LIMIT, "qk_gguf_llama: layers array too small");
    const int kv = c.dim / c.heads * c.kv_heads;
    auto get = [&](const std::string &name, bool quant, int64_t d0, int64_t d1, int &type, const void *&ptr) {
        qk_gguf_tensor t{};
        if (int s = qk_gguf_find_tensor(g, name.c_str(), &t)) return s;
        const bool type_ok = quant ? (t.type == QK_TYPE_Q4_K || t.type == QK_TYPE_Q6_K) : t.type == 0;
        if (!type_ok)
            return qk::fail(QK_ERR_TYPE, "qk_gguf_llama: unexpected storage type " + std::to_string(t.type) + " of " +
                                             name);
        const bool dims_ok = quant ? (t.n_dims == 2 && t.dims[0] == d0 && t.dims[1] == d1)
                                   : (t.n_dims == 1 && t.dims[0] == d0);
        if (!dims_ok) return qk::fail(QK_ERR_SHAPE, "qk_gguf_llama: unexpected dimensions of " + name);
        type = t.type;
        ptr = t.device;
        return QK_OK;
    };
    int f32 = 0;
    const void *p = nullptr;
    qk_llama_weights out{};
    if ((st = get("token_embd.weight", true, c.dim, c.vocab, out.embd_type, out.token_embd))) return st;
    if ((st = get("output_norm.weight", false, c.dim, 0, f32, p))) return st;
    out.output_norm = static_cast<const float *>(p);
    if (g->index.count("output.weight")) {
        if ((st = get("output.weight", true, c.dim, c.vocab, out.output_type, out.output))) return st;
    }
    for (int l = 0; l < c.layers; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        qk_llama_layer &L = layers[l];
        L = qk_llama_layer{};
        if ((st = get(b + "attn_norm.weight", false, c.dim, 0, f32, p))) return st;
        L.attn_norm = static_cast<const float *>(p);
        if ((st = get(b + "ffn_norm.weight", false, c.dim, 0, f32, p))) return st;
        L.ffn_norm = static_cast<const float *>(p);
        if ((st = get(b + "attn_q.weight", true, c.dim, c.dim, L.q_type, L.q)) ||
            (st = get(b + "attn_k.weight", true, c.dim, kv, L.k_type, L.k)) ||
            (st = get(b + "attn_v.weight", true, c.dim, kv, L.v_type, L.v)) ||
            (st = get(b + "attn_output.weight", true, c.dim, c.dim, L.o_type, L.o)) ||
            (st = get(b + "ffn_gate.weight", true, c.dim, c.hidden, L.gate_type, L.gate)) ||
            (st = get(b + "ffn_up.weight", true, c.dim, c.hidden, L.up_type, L.up)) ||
            (st = get(b + "ffn_down.weight", true, c.hidden, c.dim, L.down_type, L.down)))
            return st;
    }
    out.layers = layers;
    *cfg = c;
    *w = out;
    return qk::ok();
}

}  // extern "C"
