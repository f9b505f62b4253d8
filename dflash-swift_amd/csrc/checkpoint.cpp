/*
 * checkpoint.cpp -- MLX quantised checkpoints (safetensors) into device buffers.
 *
 * The on-disk format the fast kernel consumes, loaded without any repacking: for every
 * quantised layer P the file holds P.weight (U32 [out][in*bits/32], element 0 in the low
 * bits), P.scales and P.biases ([out][in/group_size], the model dtype) and optionally the
 * linear bias P.bias ([out]).  A layer is quantised when P.scales exists; its bits and group
 * size come from config.json's "quantization" object (per-layer entries keyed by P override
 * the top-level group_size / bits).  This is the rule MLX's loaders apply before building
 * QuantizedLinear modules, whose fields SmallMQuantizedLinear shares
 * (Sources/DFlashKit/SmallMQuantizedMatmul.swift:245-248); the model load itself is
 * loadModel, reached at Sources/dflash-bench/main.swift:26.
 *
 * safetensors layout: 8 bytes little-endian header length L, L bytes of JSON mapping each
 * tensor name to {"dtype", "shape", "data_offsets": [begin, end]} (offsets relative to the
 * byte after the header; an optional "__metadata__" object of strings), then the data.
 *
 * Device loading reads each shard in file order through two pinned staging buffers: while
 * one buffer's copies run on the stream, the next range is read into the other, by up to 8
 * threads in 4 MB pieces.  All of a
 * load's tensors go into one device allocation (256-byte aligned pieces) that the
 * checkpoint owns until it is closed.
 */
#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "json_min.h"
#include "qmm_internal.h"

using dfq::fail;

namespace {

struct DtypeName {
    const char* name;
    dfq_st_dtype code;
    int size;
};
const DtypeName kDtypes[] = {
    {"BOOL", DFQ_ST_BOOL, 1},   {"U8", DFQ_ST_U8, 1},           {"I8", DFQ_ST_I8, 1},
    {"I16", DFQ_ST_I16, 2},     {"U16", DFQ_ST_U16, 2},         {"F16", DFQ_ST_F16, 2},
    {"BF16", DFQ_ST_BF16, 2},   {"I32", DFQ_ST_I32, 4},         {"U32", DFQ_ST_U32, 4},
    {"F32", DFQ_ST_F32, 4},     {"I64", DFQ_ST_I64, 8},         {"U64", DFQ_ST_U64, 8},
    {"F64", DFQ_ST_F64, 8},     {"F8_E5M2", DFQ_ST_F8_E5M2, 1}, {"F8_E4M3", DFQ_ST_F8_E4M3, 1},
};

struct Tensor {
    std::string name;
    dfq_st_dtype dtype;
    int esize;
    std::vector<int64_t> shape;
    int shard;
    uint64_t offset;  // absolute byte offset in the shard file
    uint64_t nbytes;
};

struct Shard {
    std::string path;
    int fd = -1;
    uint64_t size = 0;
};

struct QuantParams {
    bool set = false;
    bool disabled = false;  // a per-layer entry of false
    int bits = 0, group_size = 0;
    std::string mode = "affine";
};

struct Layer {
    std::string prefix;
    int w = -1, s = -1, b = -1, bias = -1;  // tensor indices
    int out_features = 0, in_features = 0, bits = 0, group_size = 0;
    dfq_dtype dtype = DFQ_BF16;
    std::string problem;  // empty: loadable
};

bool read_all(int fd, void* dst, size_t n, uint64_t off) {
    char* p = (char*)dst;
    while (n) {
        const ssize_t r = pread(fd, p, n, (off_t)off);
        if (r < 0) {
            if (errno == EINTR) continue;
            return false;
        }
        if (r == 0) return false;
        p += r;
        n -= (size_t)r;
        off += (uint64_t)r;
    }
    return true;
}

bool ends_with(const std::string& s, const char* suf) {
    const size_t n = std::strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

bool read_text_file(const std::string& path, std::string* out) {
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return false;
    struct stat st;
    bool ok = fstat(fd, &st) == 0 && st.st_size >= 0 && st.st_size < (64 << 20);
    if (ok) {
        out->resize((size_t)st.st_size);
        ok = read_all(fd, &(*out)[0], out->size(), 0);
    }
    close(fd);
    return ok;
}

/* A "quantization" entry: an object whose group_size / bits / mode override `base`, or
 * false (the layer is not quantised). */
bool parse_quant_entry(const dfq::JsonValue& v, const QuantParams& base, QuantParams* q) {
    if (v.kind == dfq::JsonValue::Bool && !v.b) {
        *q = base;
        q->set = true;
        q->disabled = true;
        return true;
    }
    if (v.kind != dfq::JsonValue::Object) return false;
    *q = base;
    const dfq::JsonValue* gs = v.find("group_size");
    const dfq::JsonValue* bits = v.find("bits");
    const dfq::JsonValue* mode = v.find("mode");
    if (gs && gs->is_int) q->group_size = (int)gs->i;
    if (bits && bits->is_int) q->bits = (int)bits->i;
    if (mode && mode->kind == dfq::JsonValue::String) q->mode = mode->str;
    q->disabled = false;
    q->set = q->bits > 0 && q->group_size > 0;
    return q->set;
}

}  // namespace

struct dfq_checkpoint {
    std::vector<Shard> shards;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int> by_name;
    std::string format;  // __metadata__ "format" of the first shard that has one
    QuantParams dflt;
    std::unordered_map<std::string, QuantParams> per_layer;
    std::vector<Layer> layers;
    std::vector<std::pair<int, void*>> arenas;  // (device, allocation)

    ~dfq_checkpoint() {
        for (auto& a : arenas) {
            int cur = -1;
            if (hipGetDevice(&cur) == hipSuccess && cur != a.first) (void)hipSetDevice(a.first);
            (void)hipFree(a.second);
            if (cur >= 0 && cur != a.first) (void)hipSetDevice(cur);
        }
        for (auto& s : shards)
            if (s.fd >= 0) close(s.fd);
    }

    dfq_status add_shard(const std::string& path);
    void resolve_layers();
    void resolve(Layer* L) const;
};

dfq_status dfq_checkpoint::add_shard(const std::string& path) {
    Shard sh;
    sh.path = path;
    sh.fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (sh.fd < 0) return fail(DFQ_ERR_INVALID_ARGUMENT, "cannot open %s: %s", path.c_str(),
                               std::strerror(errno));
    struct stat st;
    if (fstat(sh.fd, &st) != 0) {
        close(sh.fd);
        return fail(DFQ_ERR_INVALID_ARGUMENT, "cannot stat %s", path.c_str());
    }
    sh.size = (uint64_t)st.st_size;
    const int idx = (int)shards.size();
    shards.push_back(sh);  // closed by the destructor from here on
    unsigned char len8[8];
    if (sh.size < 8 || !read_all(sh.fd, len8, 8, 0))
        return fail(DFQ_ERR_UNSUPPORTED, "%s: too short for a safetensors header", path.c_str());
    uint64_t hlen = 0;
    for (int k = 7; k >= 0; --k) hlen = (hlen << 8) | len8[k];
    if (hlen > (100ull << 20) || 8 + hlen > sh.size)
        return fail(DFQ_ERR_UNSUPPORTED, "%s: header length %llu does not fit the file",
                    path.c_str(), (unsigned long long)hlen);
    std::string hdr((size_t)hlen, '\0');
    if (hlen && !read_all(sh.fd, &hdr[0], (size_t)hlen, 8))
        return fail(DFQ_ERR_UNSUPPORTED, "%s: short read of the header", path.c_str());
    dfq::JsonValue root;
    std::string err;
    dfq::JsonParser jp(hdr.data(), hdr.size());
    if (!jp.parse(&root, &err))
        return fail(DFQ_ERR_UNSUPPORTED, "%s: header is not JSON (%s)", path.c_str(), err.c_str());
    if (root.kind != dfq::JsonValue::Object)
        return fail(DFQ_ERR_UNSUPPORTED, "%s: header is not a JSON object", path.c_str());
    const uint64_t data0 = 8 + hlen;
    for (const auto& m : root.obj) {
        if (m.first == "__metadata__") {
            if (m.second.kind != dfq::JsonValue::Object)
                return fail(DFQ_ERR_UNSUPPORTED, "%s: __metadata__ is not an object", path.c_str());
            const dfq::JsonValue* f = m.second.find("format");
            if (f && f->kind == dfq::JsonValue::String && format.empty()) format = f->str;
            continue;
        }
        const char* nm = m.first.c_str();
        const dfq::JsonValue& v = m.second;
        const dfq::JsonValue* dt = v.kind == dfq::JsonValue::Object ? v.find("dtype") : nullptr;
        const dfq::JsonValue* shp = v.kind == dfq::JsonValue::Object ? v.find("shape") : nullptr;
        const dfq::JsonValue* offs =
            v.kind == dfq::JsonValue::Object ? v.find("data_offsets") : nullptr;
        if (!dt || dt->kind != dfq::JsonValue::String || !shp ||
            shp->kind != dfq::JsonValue::Array || !offs || offs->kind != dfq::JsonValue::Array ||
            offs->arr.size() != 2)
            return fail(DFQ_ERR_UNSUPPORTED, "%s: entry %s lacks dtype / shape / data_offsets",
                        path.c_str(), nm);
        Tensor t;
        t.name = m.first;
        t.shard = idx;
        t.esize = 0;
        for (const auto& d : kDtypes)
            if (dt->str == d.name) {
                t.dtype = d.code;
                t.esize = d.size;
            }
        if (!t.esize)
            return fail(DFQ_ERR_UNSUPPORTED, "%s: tensor %s has unsupported dtype %s",
                        path.c_str(), nm, dt->str.c_str());
        uint64_t count = 1;
        for (const auto& d : shp->arr) {
            if (!d.is_int || d.i < 0)
                return fail(DFQ_ERR_UNSUPPORTED, "%s: tensor %s has a bad shape", path.c_str(), nm);
            t.shape.push_back(d.i);
            if (d.i && count > UINT64_MAX / (uint64_t)d.i)
                return fail(DFQ_ERR_UNSUPPORTED, "%s: tensor %s is too large", path.c_str(), nm);
            count *= (uint64_t)d.i;
        }
        if (t.shape.size() > 8)
            return fail(DFQ_ERR_UNSUPPORTED, "%s: tensor %s has more than 8 dimensions",
                        path.c_str(), nm);
        const dfq::JsonValue& b = offs->arr[0];
        const dfq::JsonValue& e = offs->arr[1];
        if (!b.is_int || !e.is_int || b.i < 0 || e.i < b.i)
            return fail(DFQ_ERR_UNSUPPORTED, "%s: tensor %s has bad data_offsets", path.c_str(), nm);
        t.nbytes = (uint64_t)(e.i - b.i);
        if (count > UINT64_MAX / (uint64_t)t.esize || count * (uint64_t)t.esize != t.nbytes)
            return fail(DFQ_ERR_UNSUPPORTED, "%s: tensor %s holds %llu bytes, its shape needs %llu",
                        path.c_str(), nm, (unsigned long long)t.nbytes,
                        (unsigned long long)(count * (uint64_t)t.esize));
        t.offset = data0 + (uint64_t)b.i;
        if ((uint64_t)e.i > sh.size - data0)
            return fail(DFQ_ERR_UNSUPPORTED, "%s: tensor %s runs past the end of the file",
                        path.c_str(), nm);
        if (by_name.count(t.name))
            return fail(DFQ_ERR_UNSUPPORTED, "tensor %s appears twice (second copy in %s)", nm,
                        path.c_str());
        by_name.emplace(t.name, (int)tensors.size());
        tensors.push_back(std::move(t));
    }
    return DFQ_OK;
}

/* Checks one layer's tensors against its bits / group size; sets the shape or a problem. */
void dfq_checkpoint::resolve(Layer* L) const {
    L->problem.clear();
    auto it = per_layer.find(L->prefix);
    const QuantParams& q = it != per_layer.end() ? it->second : dflt;
    char buf[256];
    auto bad = [&](const char* fmt, auto... args) {
        std::snprintf(buf, sizeof buf, fmt, args...);
        L->problem = buf;
    };
    if (!q.set) return bad("%s", "no bits / group size (config.json quantization, or set)");
    if (q.disabled) return bad("%s", "quantization is off for this layer");
    if (q.mode != "affine") return bad("mode \"%s\" is not affine", q.mode.c_str());
    L->bits = q.bits;
    L->group_size = q.group_size;
    if (q.bits != 2 && q.bits != 4 && q.bits != 8) return bad("bits %d (2, 4 or 8 supported)", q.bits);
    if (q.group_size <= 0) return bad("group size %d", q.group_size);
    const Tensor& w = tensors[L->w];
    const Tensor& s = tensors[L->s];
    if (w.dtype != DFQ_ST_U32 || w.shape.size() != 2) return bad("%s", "weight is not a 2-D U32 tensor");
    if (s.shape.size() != 2) return bad("%s", "scales is not 2-D");
    if (s.dtype != DFQ_ST_BF16 && s.dtype != DFQ_ST_F16 && s.dtype != DFQ_ST_F32)
        return bad("%s", "scales dtype is not BF16, F16 or F32");
    L->dtype = s.dtype == DFQ_ST_BF16 ? DFQ_BF16 : s.dtype == DFQ_ST_F16 ? DFQ_F16 : DFQ_F32;
    const int64_t N = w.shape[0], words = w.shape[1];
    const int64_t K = words * 32 / q.bits;
    if (words * 32 % q.bits) return bad("weight row of %lld words is not whole elements", (long long)words);
    if (N != s.shape[0]) return bad("weight has %lld rows, scales %lld", (long long)N, (long long)s.shape[0]);
    if (K % q.group_size || K / q.group_size != s.shape[1])
        return bad("in_features %lld with group size %d needs %lld groups, scales has %lld",
                   (long long)K, q.group_size, (long long)(K / q.group_size), (long long)s.shape[1]);
    if (L->b < 0) return bad("%s", "affine layer without biases");
    const Tensor& b = tensors[L->b];
    if (b.dtype != s.dtype || b.shape != s.shape) return bad("%s", "biases differ from scales in dtype or shape");
    if (L->bias >= 0) {
        const Tensor& lb = tensors[L->bias];
        if (lb.dtype != s.dtype || lb.shape.size() != 1 || lb.shape[0] != N)
            return bad("%s", "bias is not [out_features] in the scales dtype");
    }
    if (N > INT32_MAX || K > INT32_MAX) return bad("%s", "too large");
    L->out_features = (int)N;
    L->in_features = (int)K;
}

void dfq_checkpoint::resolve_layers() {
    layers.clear();
    for (size_t i = 0; i < tensors.size(); ++i) {
        const std::string& nm = tensors[i].name;
        if (!ends_with(nm, ".scales")) continue;
        Layer L;
        L.prefix = nm.substr(0, nm.size() - 7);
        L.s = (int)i;
        auto f = [&](const char* suf) {
            auto it = by_name.find(L.prefix + suf);
            return it == by_name.end() ? -1 : it->second;
        };
        L.w = f(".weight");
        if (L.w < 0) continue;  // scales without a packed weight: not a quantised layer
        L.b = f(".biases");
        L.bias = f(".bias");
        layers.push_back(L);
    }
    std::sort(layers.begin(), layers.end(),
              [](const Layer& a, const Layer& b) { return a.prefix < b.prefix; });
    for (auto& L : layers) resolve(&L);
}

namespace {

dfq_status open_dir(dfq_checkpoint* ck, const std::string& dir) {
    std::vector<std::string> files, any;
    DIR* d = opendir(dir.c_str());
    if (!d) return fail(DFQ_ERR_INVALID_ARGUMENT, "cannot list %s", dir.c_str());
    while (dirent* e = readdir(d)) {
        const std::string nm = e->d_name;
        if (!ends_with(nm, ".safetensors")) continue;
        any.push_back(nm);
        if (nm.compare(0, 5, "model") == 0) files.push_back(nm);
    }
    closedir(d);
    /* the shards MLX's loaders read: model*.safetensors, else every *.safetensors */
    if (files.empty()) files = any;
    if (files.empty())
        return fail(DFQ_ERR_INVALID_ARGUMENT, "no .safetensors files in %s", dir.c_str());
    std::sort(files.begin(), files.end());
    for (const auto& f : files)
        if (dfq_status s = ck->add_shard(dir + "/" + f)) return s;
    std::string cfg;
    if (read_text_file(dir + "/config.json", &cfg)) {
        dfq::JsonValue root;
        std::string err;
        dfq::JsonParser jp(cfg.data(), cfg.size());
        if (!jp.parse(&root, &err))
            return fail(DFQ_ERR_UNSUPPORTED, "%s/config.json is not JSON (%s)", dir.c_str(),
                        err.c_str());
        const dfq::JsonValue* q = root.kind == dfq::JsonValue::Object ? root.find("quantization")
                                                                      : nullptr;
        if (!q && root.kind == dfq::JsonValue::Object) q = root.find("quantization_config");
        if (q && q->kind == dfq::JsonValue::Object) {
            QuantParams top;
            if (!parse_quant_entry(*q, QuantParams{}, &top)) top = QuantParams{};
            ck->dflt = top;
            for (const auto& m : q->obj) {
                if (m.second.kind != dfq::JsonValue::Object &&
                    m.second.kind != dfq::JsonValue::Bool)
                    continue;
                QuantParams p;
                if (parse_quant_entry(m.second, top, &p)) ck->per_layer[m.first] = p;
            }
        }
    }
    return DFQ_OK;
}

}  // namespace

extern "C" {

dfq_status dfq_checkpoint_open(const char* path, dfq_checkpoint** out) {
    if (!path || !out) return fail(DFQ_ERR_INVALID_ARGUMENT, "null path or out");
    *out = nullptr;
    struct stat st;
    if (stat(path, &st) != 0)
        return fail(DFQ_ERR_INVALID_ARGUMENT, "cannot stat %s: %s", path, std::strerror(errno));
    auto* ck = new dfq_checkpoint();
    dfq_status s = S_ISDIR(st.st_mode) ? open_dir(ck, path) : ck->add_shard(path);
    if (s) {
        delete ck;
        return s;
    }
    ck->resolve_layers();
    *out = ck;
    return DFQ_OK;
}

dfq_status dfq_checkpoint_close(dfq_checkpoint* ck) {
    delete ck;
    return DFQ_OK;
}

const char* dfq_checkpoint_format(const dfq_checkpoint* ck) {
    return ck ? ck->format.c_str() : "";
}

int dfq_checkpoint_tensor_count(const dfq_checkpoint* ck) {
    return ck ? (int)ck->tensors.size() : 0;
}

static void fill_info(const dfq_checkpoint* ck, int i, dfq_tensor_info* out) {
    const Tensor& t = ck->tensors[i];
    std::memset(out, 0, sizeof *out);
    out->name = t.name.c_str();
    out->dtype = t.dtype;
    out->ndim = (int)t.shape.size();
    for (size_t k = 0; k < t.shape.size(); ++k) out->shape[k] = t.shape[k];
    out->nbytes = t.nbytes;
    out->shard = t.shard;
    out->offset = t.offset;
}

dfq_status dfq_checkpoint_tensor(const dfq_checkpoint* ck, int index, dfq_tensor_info* out) {
    if (!ck || !out) return fail(DFQ_ERR_INVALID_ARGUMENT, "null checkpoint or out");
    if (index < 0 || index >= (int)ck->tensors.size())
        return fail(DFQ_ERR_INVALID_ARGUMENT, "tensor index %d out of range", index);
    fill_info(ck, index, out);
    return DFQ_OK;
}

dfq_status dfq_checkpoint_find(const dfq_checkpoint* ck, const char* name, dfq_tensor_info* out) {
    if (!ck || !name || !out) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    auto it = ck->by_name.find(name);
    if (it == ck->by_name.end()) return fail(DFQ_ERR_INVALID_ARGUMENT, "no tensor %s", name);
    fill_info(ck, it->second, out);
    return DFQ_OK;
}

dfq_status dfq_checkpoint_read(const dfq_checkpoint* ck, const char* name, void* dst,
                               size_t bytes) {
    if (!ck || !name || !dst) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    auto it = ck->by_name.find(name);
    if (it == ck->by_name.end()) return fail(DFQ_ERR_INVALID_ARGUMENT, "no tensor %s", name);
    const Tensor& t = ck->tensors[it->second];
    if (bytes < t.nbytes)
        return fail(DFQ_ERR_INVALID_ARGUMENT, "%s needs %llu bytes (got %zu)", name,
                    (unsigned long long)t.nbytes, bytes);
    if (!read_all(ck->shards[t.shard].fd, dst, t.nbytes, t.offset))
        return fail(DFQ_ERR_INVALID_ARGUMENT, "short read of %s", name);
    return DFQ_OK;
}

dfq_status dfq_checkpoint_set_quantization(dfq_checkpoint* ck, const char* prefix, int bits,
                                           int group_size) {
    if (!ck) return fail(DFQ_ERR_INVALID_ARGUMENT, "null checkpoint");
    QuantParams q;
    q.set = true;
    q.bits = bits;
    q.group_size = group_size;
    if (prefix) ck->per_layer[prefix] = q;
    else ck->dflt = q;
    for (auto& L : ck->layers) ck->resolve(&L);
    return DFQ_OK;
}

int dfq_checkpoint_layer_count(const dfq_checkpoint* ck) {
    return ck ? (int)ck->layers.size() : 0;
}

dfq_status dfq_checkpoint_layer(const dfq_checkpoint* ck, int index, dfq_layer_info* out) {
    if (!ck || !out) return fail(DFQ_ERR_INVALID_ARGUMENT, "null checkpoint or out");
    if (index < 0 || index >= (int)ck->layers.size())
        return fail(DFQ_ERR_INVALID_ARGUMENT, "layer index %d out of range", index);
    const Layer& L = ck->layers[index];
    std::memset(out, 0, sizeof *out);
    out->prefix = L.prefix.c_str();
    out->out_features = L.out_features;
    out->in_features = L.in_features;
    out->bits = L.bits;
    out->group_size = L.group_size;
    out->has_biases = L.b >= 0;
    out->has_bias = L.bias >= 0;
    out->dtype = L.dtype;
    out->valid = L.problem.empty();
    out->problem = L.problem.c_str();
    return DFQ_OK;
}

/* One contiguous file range and where it goes on the device. */
struct Piece {
    int shard;
    uint64_t off, len;
    char* dst;
};

static dfq_status copy_pieces(dfq_checkpoint* ck, std::vector<Piece>& pieces, size_t total,
                              hipStream_t stream) {
    std::sort(pieces.begin(), pieces.end(), [](const Piece& a, const Piece& b) {
        return a.shard != b.shard ? a.shard < b.shard : a.off < b.off;
    });
    const size_t kStage = std::min<size_t>(64u << 20, std::max<size_t>(total, 1));
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    dfq_status st = DFQ_OK;
    hipError_t e = hipSuccess;
    for (int k = 0; k < 2 && e == hipSuccess; ++k) {
        e = hipHostMalloc(&buf[k], kStage, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev[k], hipEventDisableTiming);
    }
    if (e != hipSuccess) st = fail(DFQ_ERR_HIP, "staging buffers: %s", hipGetErrorString(e));
    struct Rec {
        size_t at;
        char* dst;
        size_t n;
    };
    std::vector<Rec> recs;
    struct Read {
        int shard;
        uint64_t off;
        size_t at, n;
    };
    std::vector<Read> reads;
    constexpr size_t kReadChunk = 4u << 20;
    const size_t kReaders = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
    size_t pi = 0;
    uint64_t done_in_piece = 0;
    bool used[2] = {false, false};
    for (int cur = 0; st == DFQ_OK && pi < pieces.size(); cur ^= 1) {
        if (used[cur] && (e = hipEventSynchronize(ev[cur])) != hipSuccess) {
            st = fail(DFQ_ERR_HIP, "staging wait: %s", hipGetErrorString(e));
            break;
        }
        /* plan this buffer's ranges, then read them with several threads (pread is
         * positional, so the threads share each shard's descriptor) */
        size_t fill = 0;
        recs.clear();
        reads.clear();
        while (pi < pieces.size() && fill < kStage) {
            const Piece& p = pieces[pi];
            const size_t n = (size_t)std::min<uint64_t>(p.len - done_in_piece, kStage - fill);
            recs.push_back({fill, p.dst + done_in_piece, n});
            for (size_t k = 0; k < n; k += kReadChunk)
                reads.push_back({p.shard, p.off + done_in_piece + k, fill + k,
                                 std::min(kReadChunk, n - k)});
            fill += n;
            done_in_piece += n;
            if (done_in_piece == p.len) {
                ++pi;
                done_in_piece = 0;
            }
        }
        std::atomic<size_t> next{0};
        std::atomic<int> bad_shard{-1};
        auto reader = [&]() {
            for (size_t r; (r = next.fetch_add(1)) < reads.size();) {
                const Read& rd = reads[r];
                if (!read_all(ck->shards[rd.shard].fd, (char*)buf[cur] + rd.at, rd.n, rd.off))
                    bad_shard.store(rd.shard);
            }
        };
        const int nthr = (int)std::min<size_t>(kReaders, reads.size());
        std::vector<std::thread> pool;
        for (int k = 1; k < nthr; ++k) pool.emplace_back(reader);
        reader();
        for (auto& th : pool) th.join();
        if (bad_shard.load() >= 0) {
            st = fail(DFQ_ERR_INVALID_ARGUMENT, "short read from %s",
                      ck->shards[bad_shard.load()].path.c_str());
            break;
        }
        for (const Rec& r : recs)
            if ((e = hipMemcpyAsync(r.dst, (char*)buf[cur] + r.at, r.n, hipMemcpyHostToDevice,
                                    stream)) != hipSuccess)
                break;
        if (e == hipSuccess) e = hipEventRecord(ev[cur], stream);
        if (e != hipSuccess) st = fail(DFQ_ERR_HIP, "upload: %s", hipGetErrorString(e));
        used[cur] = true;
    }
    /* the staging buffers are freed below: every copy out of them must have finished */
    if ((e = hipStreamSynchronize(stream)) != hipSuccess && st == DFQ_OK)
        st = fail(DFQ_ERR_HIP, "upload sync: %s", hipGetErrorString(e));
    for (int k = 0; k < 2; ++k) {
        if (ev[k]) (void)hipEventDestroy(ev[k]);
        if (buf[k]) (void)hipHostFree(buf[k]);
    }
    return st;
}

dfq_status dfq_checkpoint_upload(dfq_ctx* ctx, dfq_checkpoint* ck, const char* name, void* dst,
                                 size_t bytes, void* stream) {
    if (!ctx || !ck || !name || !dst) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    auto it = ck->by_name.find(name);
    if (it == ck->by_name.end()) return fail(DFQ_ERR_INVALID_ARGUMENT, "no tensor %s", name);
    const Tensor& t = ck->tensors[it->second];
    if (bytes < t.nbytes)
        return fail(DFQ_ERR_INVALID_ARGUMENT, "%s needs %llu bytes (got %zu)", name,
                    (unsigned long long)t.nbytes, bytes);
    dfq::DeviceScope g(ctx);
    std::vector<Piece> pieces{{t.shard, t.offset, t.nbytes, (char*)dst}};
    return copy_pieces(ck, pieces, t.nbytes, (hipStream_t)stream);
}

/* Whether layer L loads into the packed layout: an affine 4/8-bit layer with biases whose
 * scales are bf16 or fp16, K a whole number of 8-group chunks, and a fast-kernel split at
 * every row count of a launch (1..16). */
static bool packs(dfq_ctx* ctx, const Layer& L) {
    size_t nb = 0;
    if (L.b < 0 || (L.dtype != DFQ_BF16 && L.dtype != DFQ_F16) ||
        dfq_packed_bytes(L.out_features, L.in_features, L.bits, L.group_size, &nb) != DFQ_OK)
        return false;
    for (int r = 1; r <= DFQ_MAXIMUM_ROWS; ++r)
        if (!dfq_qmm_supported(ctx, r, L.out_features, L.in_features, L.bits, L.group_size,
                               L.dtype, L.dtype, L.dtype))
            return false;
    return true;
}

static dfq_status load_model(dfq_ctx* ctx, dfq_checkpoint* ck, dfq_model* model,
                             int (*want)(const char* prefix, void* user), void* user,
                             void* stream, int* loaded, bool pack) {
    if (loaded) *loaded = 0;
    if (!ctx || !ck || !model) return fail(DFQ_ERR_INVALID_ARGUMENT, "null ctx, checkpoint or model");
    std::vector<const Layer*> sel;
    for (const auto& L : ck->layers) {
        if (want && !want(L.prefix.c_str(), user)) continue;
        if (!L.problem.empty())
            return fail(DFQ_ERR_UNSUPPORTED, "layer %s: %s", L.prefix.c_str(), L.problem.c_str());
        sel.push_back(&L);
    }
    if (sel.empty()) return DFQ_OK;
    /* One allocation, each array at a 256-byte aligned offset: a packed layer's packed weight
     * (slot 0) and linear bias (slot 3); any other layer's weight, scales, biases and bias as
     * stored.  A packed layer's three MLX tensors pass through a device staging buffer, a
     * batch of layers at a time, and are packed from there. */
    struct Slot {
        int tensor;
        size_t at;
    };
    const auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    std::vector<std::vector<Slot>> slots(sel.size());
    std::vector<char> packed(sel.size(), 0);
    size_t total = 0, stage_max = 0, stage_all = 0;
    for (size_t i = 0; i < sel.size(); ++i) {
        const Layer& L = *sel[i];
        packed[i] = pack && packs(ctx, L);
        if (packed[i]) {
            size_t nb = 0;
            (void)dfq_packed_bytes(L.out_features, L.in_features, L.bits, L.group_size, &nb);
            slots[i] = {{-1, total}, {-1, 0}, {-1, 0}, {L.bias, 0}};
            total += up(nb);
            if (L.bias >= 0) {
                slots[i][3].at = total;
                total += up(ck->tensors[L.bias].nbytes);
            }
            const size_t sb = up(ck->tensors[L.w].nbytes) + up(ck->tensors[L.s].nbytes) +
                              up(ck->tensors[L.b].nbytes);
            stage_max = std::max(stage_max, sb);
            stage_all += sb;
            continue;
        }
        for (int ti : {L.w, L.s, L.b, L.bias}) {
            if (ti < 0) {
                slots[i].push_back({-1, 0});
                continue;
            }
            slots[i].push_back({ti, total});
            total += up(ck->tensors[ti].nbytes);
        }
    }
    dfq::DeviceScope g(ctx);
    void* arena = nullptr;
    void* stage = nullptr;
    const size_t stage_bytes = std::max(stage_max, std::min(stage_all, (size_t)1 << 30));
    hipError_t e = hipMalloc(&arena, total);
    if (e != hipSuccess)
        return fail(DFQ_ERR_HIP, "device allocation of %zu bytes: %s", total, hipGetErrorString(e));
    if (stage_all && (e = hipMalloc(&stage, stage_bytes)) != hipSuccess) {
        (void)hipFree(arena);
        return fail(DFQ_ERR_HIP, "packing stage of %zu bytes: %s", stage_bytes,
                    hipGetErrorString(e));
    }
    std::vector<Piece> pieces;
    for (auto& ls : slots)
        for (const Slot& s : ls)
            if (s.tensor >= 0) {
                const Tensor& t = ck->tensors[s.tensor];
                pieces.push_back({t.shard, t.offset, t.nbytes, (char*)arena + s.at});
            }
    dfq_status st = pieces.empty() ? DFQ_OK : copy_pieces(ck, pieces, total, (hipStream_t)stream);
    /* packed layers: fill the stage with as many as fit, pack them, repeat (copy_pieces
     * returns once its copies are done; the packs run on the same stream before the next
     * batch's copies overwrite the stage) */
    for (size_t i = 0; st == DFQ_OK && i < sel.size();) {
        std::vector<Piece> batch;
        std::vector<std::pair<size_t, size_t>> layers;  // (layer, stage offset)
        size_t fill = 0;
        for (; i < sel.size(); ++i) {
            if (!packed[i]) continue;
            const Layer& L = *sel[i];
            const size_t sb = up(ck->tensors[L.w].nbytes) + up(ck->tensors[L.s].nbytes) +
                              up(ck->tensors[L.b].nbytes);
            if (fill + sb > stage_bytes) break;
            layers.push_back({i, fill});
            for (int ti : {L.w, L.s, L.b}) {
                const Tensor& t = ck->tensors[ti];
                batch.push_back({t.shard, t.offset, t.nbytes, (char*)stage + fill});
                fill += up(t.nbytes);
            }
        }
        if (batch.empty()) break;
        st = copy_pieces(ck, batch, fill, (hipStream_t)stream);
        for (size_t k = 0; st == DFQ_OK && k < layers.size(); ++k) {
            const Layer& L = *sel[layers[k].first];
            char* base = (char*)stage + layers[k].second;
            const size_t ws = up(ck->tensors[L.w].nbytes), ss = up(ck->tensors[L.s].nbytes);
            st = dfq_pack_weights(ctx, (const uint32_t*)base, base + ws, base + ws + ss,
                                  L.out_features, L.in_features, L.bits, L.group_size,
                                  (char*)arena + slots[layers[k].first][0].at, stream);
        }
    }
    if (stage) {
        if ((e = hipStreamSynchronize((hipStream_t)stream)) != hipSuccess && st == DFQ_OK)
            st = fail(DFQ_ERR_HIP, "packing: %s", hipGetErrorString(e));
        (void)hipFree(stage);
    }
    std::vector<dfq_linear*> lins;
    for (size_t i = 0; st == DFQ_OK && i < sel.size(); ++i) {
        const Layer& L = *sel[i];
        auto at = [&](int k) -> void* {
            return slots[i][k].tensor < 0 ? nullptr : (char*)arena + slots[i][k].at;
        };
        dfq_linear_desc d{};
        d.bias = at(3);
        d.out_features = L.out_features;
        d.in_features = L.in_features;
        d.bits = L.bits;
        d.group_size = L.group_size;
        d.mode_affine = 1;
        d.dtype = L.dtype;
        dfq_linear* lin = nullptr;
        if (packed[i]) {
            st = dfq::make_packed_linear(ctx, d, (char*)arena + slots[i][0].at, &lin);
        } else {
            d.weight = (const uint32_t*)at(0);
            d.scales = at(1);
            d.biases = at(2);
            st = dfq_linear_create(ctx, &d, &lin);
        }
        if (st == DFQ_OK) lins.push_back(lin);
    }
    if (st != DFQ_OK) {
        for (dfq_linear* l : lins) dfq_linear_destroy(l);
        (void)hipFree(arena);
        return st;
    }
    ck->arenas.emplace_back(dfq::ctx_device(ctx), arena);
    for (size_t i = 0; i < sel.size(); ++i)
        if ((st = dfq_model_set_leaf(model, sel[i]->prefix.c_str(), lins[i])) != DFQ_OK) {
            for (size_t j = i; j < sel.size(); ++j) dfq_linear_destroy(lins[j]);
            return st;
        }
    if (loaded) *loaded = (int)sel.size();
    return DFQ_OK;
}

dfq_status dfq_checkpoint_load_model(dfq_ctx* ctx, dfq_checkpoint* ck, dfq_model* model,
                                     int (*want)(const char* prefix, void* user), void* user,
                                     void* stream, int* loaded) {
    return load_model(ctx, ck, model, want, user, stream, loaded, false);
}

dfq_status dfq_checkpoint_load_model_packed(dfq_ctx* ctx, dfq_checkpoint* ck, dfq_model* model,
                                            int (*want)(const char* prefix, void* user),
                                            void* user, void* stream, int* loaded) {
    return load_model(ctx, ck, model, want, user, stream, loaded, true);
}

}  // extern "C"
