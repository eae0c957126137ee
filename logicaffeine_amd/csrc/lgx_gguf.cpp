// lgx_gguf.cpp -- reader of Q8_0 Qwen2 checkpoints in the GGUF container.
//
// GGUF (the llama.cpp model file, format version 2 and 3) is a little-endian
// stream:
//   magic "GGUF", version u32, tensor count u64, metadata count u64,
//   metadata: key (u64 length + bytes), value type u32, value
//     (u8 i8 u16 i16 u32 i32 f32 bool string array u64 i64 f64 = types 0..12;
//      an array is element type u32 + count u64 + elements),
//   tensor infos: name, n_dims u32, dims u64[n_dims] (dims[0] the row length),
//     ggml type u32, offset u64 (from the data section),
//   padding to general.alignment (default 32), then the data section.
// Tensor types read here: F32 (0), F16 (1) and Q8_0 (8; also for
// token_embd, as llama.cpp's Q8_0 conversion stores it): blocks of 32
// values stored as a binary16 scale d followed by 32 int8 quants (34 bytes),
// the same block as the Q8_0 format the kernels use, so a row of Q8_0 blocks
// splits into the row-major quants/scales that lgx_q8_repack_t16 takes.
//
// Qwen2 tensor names (the llama.cpp convention): token_embd.weight,
// output_norm.weight, output.weight (absent when the embedding is tied),
// blk.N.{attn_norm, attn_q, attn_k, attn_v, attn_output, ffn_norm, ffn_gate,
// ffn_up, ffn_down}.weight and blk.N.attn_{q,k,v}.bias.  Qwen2 files keep the
// Hugging Face (rotate-half) order of the query/key rows, the RoPE pairing
// the kernels use.  The reference has no model format (it has no model);
// this reader is the on-disk path next to the seeded generator.
#include "lgx_gguf.h"

#include <cstring>

#include "lgx_internal.h"

using namespace lgxi;

namespace lgxf {

namespace {
// A string read from the file, as it appears in an error message: printable
// ASCII only (other bytes as '?'), at most 64 characters.
std::string shown(const std::string& s) {
    std::string o;
    for (size_t i = 0; i < s.size() && i < 64; ++i) {
        const unsigned char ch = (unsigned char)s[i];
        o += ch >= 0x20 && ch < 0x7f ? (char)ch : '?';
    }
    if (s.size() > 64) o += "...";
    return o;
}

enum : uint32_t {
    GT_U8 = 0, GT_I8, GT_U16, GT_I16, GT_U32, GT_I32, GT_F32, GT_BOOL, GT_STRING, GT_ARRAY,
    GT_U64, GT_I64, GT_F64
};

struct Reader {
    FILE* f;
    bool ok = true;
    template <class T>
    T get() {
        T v{};
        if (ok && fread(&v, sizeof(T), 1, f) != 1) ok = false;
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (1ull << 30)) {
            ok = false;
            return {};
        }
        std::string s(n, '\0');
        if (n && fread(&s[0], 1, n, f) != n) ok = false;
        return s;
    }
    void skip(uint64_t n) {
        if (ok && fseeko(f, (off_t)n, SEEK_CUR) != 0) ok = false;
    }
};

size_t scalar_size(uint32_t t) {
    switch (t) {
        case GT_U8: case GT_I8: case GT_BOOL: return 1;
        case GT_U16: case GT_I16: return 2;
        case GT_U32: case GT_I32: case GT_F32: return 4;
        case GT_U64: case GT_I64: case GT_F64: return 8;
        default: return 0;
    }
}

// One metadata value: numbers kept (as double / int64), strings kept,
// arrays skipped.
bool read_value(Reader& r, uint32_t type, Meta& m, int depth = 0) {
    m.type = type;
    switch (type) {
        case GT_U8: m.i = r.get<uint8_t>(); break;
        case GT_I8: m.i = r.get<int8_t>(); break;
        case GT_U16: m.i = r.get<uint16_t>(); break;
        case GT_I16: m.i = r.get<int16_t>(); break;
        case GT_U32: m.i = r.get<uint32_t>(); break;
        case GT_I32: m.i = r.get<int32_t>(); break;
        case GT_U64: m.i = (int64_t)r.get<uint64_t>(); break;
        case GT_I64: m.i = r.get<int64_t>(); break;
        case GT_BOOL: m.i = r.get<uint8_t>(); break;
        case GT_F32: m.f = r.get<float>(); m.i = (int64_t)m.f; break;
        case GT_F64: m.f = r.get<double>(); m.i = (int64_t)m.f; break;
        case GT_STRING: m.s = r.str(); break;
        case GT_ARRAY: {
            if (depth > 0) return false;
            const uint32_t et = r.get<uint32_t>();
            const uint64_t n = r.get<uint64_t>();
            if (!r.ok) return false;
            if (et == GT_STRING) {
                for (uint64_t i = 0; i < n && r.ok; ++i) r.skip(r.get<uint64_t>());
            } else {
                const size_t es = scalar_size(et);
                if (!es) return false;
                r.skip(n * es);
            }
            break;
        }
        default: return false;
    }
    if (type == GT_U8 || type == GT_I8 || type == GT_U16 || type == GT_I16 || type == GT_U32 ||
        type == GT_I32 || type == GT_U64 || type == GT_I64 || type == GT_BOOL)
        m.f = (double)m.i;
    return r.ok;
}
}  // namespace

lgx_status Gguf::open(const char* p) {
    path = p ? p : "";
    if (!p) return fail(LGX_NULL_POINTER, "NULL path");
    f = fopen(p, "rb");
    if (!f) return fail(LGX_MODULE_LOAD_FAILED, "cannot open %s", p);
    Reader r{f};
    const uint32_t magic = r.get<uint32_t>();
    if (!r.ok || magic != 0x46554747u)
        return fail(LGX_MODULE_LOAD_FAILED, "%s: not a GGUF file (magic %08x)", p, magic);
    const uint32_t version = r.get<uint32_t>();
    if (version != 2 && version != 3)
        return fail(LGX_UNSUPPORTED, "%s: GGUF version %u (2 and 3 are read)", p, version);
    const uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
    if (!r.ok || nt > (1u << 24) || nkv > (1u << 24))
        return fail(LGX_MODULE_LOAD_FAILED, "%s: truncated or corrupt header", p);
    for (uint64_t i = 0; i < nkv; ++i) {
        std::string key = r.str();
        const uint32_t type = r.get<uint32_t>();
        Meta m;
        if (!r.ok || !read_value(r, type, m))
            return fail(LGX_MODULE_LOAD_FAILED, "%s: bad metadata entry %llu (%s)", p,
                        (unsigned long long)i, shown(key).c_str());
        meta[key] = m;
    }
    for (uint64_t i = 0; i < nt; ++i) {
        TensorInfo t;
        t.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (!r.ok || nd == 0 || nd > 4)
            return fail(LGX_MODULE_LOAD_FAILED, "%s: bad tensor info %llu", p, (unsigned long long)i);
        for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(r.get<uint64_t>());
        t.type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        if (!r.ok) return fail(LGX_MODULE_LOAD_FAILED, "%s: truncated tensor infos", p);
        tensors[t.name] = t;
    }
    auto al = meta.find("general.alignment");
    alignment = al != meta.end() && al->second.i > 0 ? (uint64_t)al->second.i : 32;
    const off_t here = ftello(f);
    if (here < 0) return fail(LGX_MODULE_LOAD_FAILED, "%s: ftello failed", p);
    data_start = ((uint64_t)here + alignment - 1) / alignment * alignment;
    if (fseeko(f, 0, SEEK_END) != 0) return fail(LGX_MODULE_LOAD_FAILED, "%s: seek failed", p);
    const off_t end = ftello(f);
    if (end < 0) return fail(LGX_MODULE_LOAD_FAILED, "%s: ftello failed", p);
    file_size = (uint64_t)end;
    return check_extents();
}

// Bytes of a tensor of `elems` values of `type` (0 for a type not read here).
static uint64_t tensor_bytes(uint32_t type, uint64_t elems) {
    switch (type) {
        case GGML_F32: return elems * 4;
        case GGML_F16: return elems * 2;
        case GGML_Q8_0: return elems / 32 * 34;
        default: return 0;
    }
}

// Element count of a tensor's dims, or false when a dim is 0 or the product
// exceeds 2^48 (far above any model tensor; keeps every byte count below
// 2^54 with no overflow).
static bool tensor_elems(const TensorInfo& t, uint64_t* out) {
    uint64_t n = 1;
    for (uint64_t d : t.dims) {
        if (d == 0 || d > (1ull << 48) || __builtin_mul_overflow(n, d, &n) || n > (1ull << 48))
            return false;
    }
    *out = n;
    return true;
}

// Every tensor of a type this reader knows lies inside the data section:
// offset + bytes <= file_size - data_start, compared without wrap-around.
lgx_status Gguf::check_extents() const {
    if (data_start > file_size)
        return fail(LGX_MODULE_LOAD_FAILED, "%s: no data section", path.c_str());
    const uint64_t room = file_size - data_start;
    for (const auto& kv : tensors) {
        const TensorInfo& t = kv.second;
        uint64_t elems = 0;
        if (!tensor_elems(t, &elems))
            return fail(LGX_MODULE_LOAD_FAILED, "%s: tensor %s has invalid dims", path.c_str(),
                        shown(t.name).c_str());
        if (t.type == GGML_Q8_0 && t.dims[0] % 32 != 0)
            return fail(LGX_MODULE_LOAD_FAILED, "%s: Q8_0 tensor %s has a row of %llu values",
                        path.c_str(), shown(t.name).c_str(), (unsigned long long)t.dims[0]);
        const uint64_t nbytes = tensor_bytes(t.type, elems);
        if (nbytes > room || t.offset > room - nbytes)
            return fail(LGX_MODULE_LOAD_FAILED, "%s: tensor %s runs past the end of the file",
                        path.c_str(), shown(t.name).c_str());
    }
    return LGX_OK;
}

Gguf::~Gguf() {
    if (f) fclose(f);
}

const Meta* Gguf::find(const std::string& key) const {
    auto it = meta.find(key);
    return it == meta.end() ? nullptr : &it->second;
}

const TensorInfo* Gguf::tensor(const std::string& name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? nullptr : &it->second;
}

// The tensor `name` with shape rows x cols (dims[0] = cols) and `type`,
// positioned for reading.
lgx_status Gguf::seek(const std::string& name, uint32_t type, int64_t rows, int64_t cols) const {
    const TensorInfo* t = tensor(name);
    if (!t)
        return fail(LGX_INVALID_ARGUMENT, "%s: tensor %s missing", path.c_str(), shown(name).c_str());
    // open() checked the dims (product <= 2^48) and the extent of the tensor
    const int64_t d0 = (int64_t)t->dims[0];
    int64_t rest = 1;
    for (size_t i = 1; i < t->dims.size(); ++i) rest *= (int64_t)t->dims[i];
    if (t->type != type)
        return fail(LGX_UNSUPPORTED, "%s: tensor %s has ggml type %u (expected %u)", path.c_str(),
                    shown(name).c_str(), t->type, type);
    if (d0 != cols || rest != rows)
        return fail(LGX_INVALID_ARGUMENT, "%s: tensor %s is %lld x %lld (expected %lld x %lld)",
                    path.c_str(), shown(name).c_str(), (long long)rest, (long long)d0, (long long)rows,
                    (long long)cols);
    if (fseeko(f, (off_t)(data_start + t->offset), SEEK_SET) != 0)
        return fail(LGX_MODULE_LOAD_FAILED, "%s: seek to %s failed", path.c_str(),
                    shown(name).c_str());
    return LGX_OK;
}

lgx_status Gguf::read_q8(const std::string& name, int64_t rows, int64_t cols, int8_t* qs,
                         uint16_t* d) const {
    if (cols % 32)
        return fail(LGX_UNSUPPORTED, "%s: row length %lld", shown(name).c_str(), (long long)cols);
    lgx_status st = seek(name, GGML_Q8_0, rows, cols);
    if (st != LGX_OK) return st;
    const int64_t nb = cols / 32;
    std::vector<uint8_t> row((size_t)nb * 34);
    for (int64_t r = 0; r < rows; ++r) {
        if (fread(row.data(), 1, row.size(), f) != row.size())
            return fail(LGX_MODULE_LOAD_FAILED, "%s: short read of %s", path.c_str(), shown(name).c_str());
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row.data() + b * 34;
            d[r * nb + b] = (uint16_t)(blk[0] | (blk[1] << 8));
            memcpy(qs + r * cols + b * 32, blk + 2, 32);
        }
    }
    return LGX_OK;
}

lgx_status Gguf::read_raw(const std::string& name, uint32_t type, int64_t rows, int64_t cols,
                          void* out) const {
    lgx_status st = seek(name, type, rows, cols);
    if (st != LGX_OK) return st;
    const size_t nbytes = (size_t)tensor_bytes(type, (uint64_t)rows * cols);
    if (fread(out, 1, nbytes, f) != nbytes)
        return fail(LGX_MODULE_LOAD_FAILED, "%s: short read of %s", path.c_str(), shown(name).c_str());
    return LGX_OK;
}

// The model shape from the metadata and tensor shapes of a Qwen2 file.
lgx_status Gguf::config(int32_t max_batch, int32_t max_seq, lgx_qwen_config* cfg) const {
    const Meta* arch = find("general.architecture");
    if (!arch || arch->type != GT_STRING)
        return fail(LGX_INVALID_ARGUMENT, "%s: no general.architecture", path.c_str());
    if (arch->s != "qwen2")
        return fail(LGX_UNSUPPORTED, "%s: architecture %s (qwen2 is read)", path.c_str(),
                    shown(arch->s).c_str());
    auto num = [&](const char* key, double* v) -> lgx_status {
        const Meta* m = find(std::string("qwen2.") + key);
        if (!m || m->type == GT_STRING || m->type == GT_ARRAY)
            return fail(LGX_INVALID_ARGUMENT, "%s: metadata qwen2.%s missing", path.c_str(), key);
        *v = m->f;
        return LGX_OK;
    };
    double L, H, I, hq, hkv;
    lgx_status st;
    if ((st = num("block_count", &L)) || (st = num("embedding_length", &H)) ||
        (st = num("feed_forward_length", &I)) || (st = num("attention.head_count", &hq)) ||
        (st = num("attention.head_count_kv", &hkv)))
        return st;
    double eps = 1e-6, theta = 1e6;
    if (num("attention.layer_norm_rms_epsilon", &eps) != LGX_OK) eps = 1e-6;
    if (num("rope.freq_base", &theta) != LGX_OK) theta = 1e6;
    g_has_error = false;
    // every number in range before the int32 conversions
    auto in = [](double v, double lo, double hi) { return v >= lo && v <= hi && v == (double)(int64_t)v; };
    if (!in(L, 1, 4096) || !in(H, 1, 1 << 20) || !in(I, 1, 1 << 22) || !in(hq, 1, 4096) ||
        !in(hkv, 1, 4096))
        return fail(LGX_INVALID_ARGUMENT, "%s: model shape out of range (layers %g, hidden %g, "
                    "ffn %g, heads %g / %g)", path.c_str(), L, H, I, hq, hkv);
    if (!(eps > 0.0 && eps < 1.0) || !(theta > 0.0 && theta < 1e30))
        return fail(LGX_INVALID_ARGUMENT, "%s: rms epsilon %g or rope base %g out of range",
                    path.c_str(), eps, theta);
    const TensorInfo* emb = tensor("token_embd.weight");
    if (!emb || emb->dims.size() != 2)
        return fail(LGX_INVALID_ARGUMENT, "%s: token_embd.weight missing", path.c_str());
    lgx_qwen_config c{};
    c.n_layers = (int32_t)L;
    c.hidden = (int32_t)H;
    c.intermediate = (int32_t)I;
    c.n_heads = (int32_t)hq;
    c.n_kv_heads = (int32_t)hkv;
    c.head_dim = c.n_heads > 0 ? c.hidden / c.n_heads : 0;
    double kl;
    if (num("attention.key_length", &kl) == LGX_OK) {
        if (!in(kl, 1, 4096))
            return fail(LGX_INVALID_ARGUMENT, "%s: key length %g out of range", path.c_str(), kl);
        c.head_dim = (int32_t)kl;
    }
    g_has_error = false;
    if (emb->dims[1] > 0x7fffffffull)
        return fail(LGX_INVALID_ARGUMENT, "%s: vocabulary of %llu rows", path.c_str(),
                    (unsigned long long)emb->dims[1]);
    c.vocab = (int32_t)emb->dims[1];
    c.tied_embedding = tensor("output.weight") ? 0 : 1;
    c.max_batch = max_batch;
    c.max_seq = max_seq;
    c.rms_eps = (float)eps;
    c.rope_theta = theta;
    c.emb_sigma = 0.0;
    if ((int64_t)emb->dims[0] != c.hidden)
        return fail(LGX_INVALID_ARGUMENT, "%s: token_embd row length %llu, hidden %d", path.c_str(),
                    (unsigned long long)emb->dims[0], c.hidden);
    if (emb->type != GGML_F16 && emb->type != GGML_Q8_0)
        return fail(LGX_UNSUPPORTED, "%s: token_embd.weight has ggml type %u (F16 and Q8_0 are read)",
                    path.c_str(), emb->type);
    *cfg = c;
    return LGX_OK;
}

}  // namespace lgxf
