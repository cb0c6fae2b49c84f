// Safetensors checkpoints (safetensors.rs) mapped read-only and fed to the
// device loaders: the decoder's and encoder's matrices go from the file
// mapping straight through the pinned staging ring into HBM (no host copy of
// the checkpoint), and the int8 packing runs on the GPU.
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "decoder.h"

namespace {

struct StTensor {
    int dtype = QASR_ST_UNKNOWN;
    std::vector<int64_t> shape;
    const uint8_t *data = nullptr;
    int64_t bytes = 0;
};

struct Mapping {
    void *base = MAP_FAILED;
    size_t size = 0;
    ~Mapping() {
        if (base != MAP_FAILED) munmap(base, size);
    }
};

int elem_size(int dtype) {
    switch (dtype) {
        case QASR_ST_F32: case QASR_ST_I32: return 4;
        case QASR_ST_F16: case QASR_ST_BF16: return 2;
        case QASR_ST_I64: return 8;
        case QASR_ST_BOOL: return 1;
        default: return 0;
    }
}

int dtype_code(const std::string &s) {     // Dtype::from_str (safetensors.rs:20-31)
    if (s == "F32") return QASR_ST_F32;
    if (s == "F16") return QASR_ST_F16;
    if (s == "BF16") return QASR_ST_BF16;
    if (s == "I32") return QASR_ST_I32;
    if (s == "I64") return QASR_ST_I64;
    if (s == "BOOL") return QASR_ST_BOOL;
    return QASR_ST_UNKNOWN;
}

// A strict reader for the header's JSON: one object of
// name -> {"dtype": s, "shape": [n...], "data_offsets": [a, b]}, plus an
// optional "__metadata__" object; unknown keys and values are skipped.
class Json {
public:
    Json(const char *p, size_t n) : p_(p), e_(p + n) {}
    std::string err;

    bool header(std::vector<std::pair<std::string, StTensor>> &out, int64_t &max_end, uint64_t data_len) {
        ws();
        if (!lit('{')) return fail("header is not a JSON object");
        ws();
        if (lit('}')) return tail();
        for (;;) {
            std::string key;
            ws();
            if (!str(key)) return fail("bad tensor name");
            ws();
            if (!lit(':')) return fail("missing ':'");
            ws();
            if (key == "__metadata__") {
                if (!skip(0)) return false;
            } else {
                StTensor t;
                if (!tensor(t, data_len, max_end)) return false;
                out.emplace_back(key, std::move(t));
            }
            ws();
            if (lit(',')) continue;
            if (lit('}')) return tail();
            return fail("expected ',' or '}'");
        }
    }

private:
    const char *p_, *e_;
    bool fail(const std::string &m) {
        if (err.empty()) err = m;
        return false;
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool lit(char c) {
        if (p_ < e_ && *p_ == c) {
            p_++;
            return true;
        }
        return false;
    }
    bool tail() {
        ws();
        return p_ == e_ ? true : fail("trailing bytes after the header object");
    }
    static int hex(char c) {
        if (c >= '0' && c <= '9') return c - '0';
        if (c >= 'a' && c <= 'f') return c - 'a' + 10;
        if (c >= 'A' && c <= 'F') return c - 'A' + 10;
        return -1;
    }
    bool u16(unsigned &v) {
        if (e_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; i++) {
            const int h = hex(p_[i]);
            if (h < 0) return false;
            v = v * 16 + (unsigned)h;
        }
        p_ += 4;
        return true;
    }
    static void utf8(std::string &s, unsigned cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool str(std::string &s) {
        if (!lit('"')) return false;
        while (p_ < e_) {
            const char c = *p_++;
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return fail("control character in a string");
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= e_) break;
            const char x = *p_++;
            switch (x) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    unsigned cp;
                    if (!u16(cp)) return fail("bad \\u escape");
                    if (cp >= 0xD800 && cp < 0xDC00) {       // surrogate pair
                        unsigned lo;
                        if (!(lit('\\') && lit('u') && u16(lo)) || lo < 0xDC00 || lo >= 0xE000)
                            return fail("unpaired surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail("unpaired surrogate");
                    }
                    utf8(s, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        return fail("unterminated string");
    }
    bool integer(int64_t &v) {
        const char *q = p_;
        bool neg = lit('-');
        if (p_ >= e_ || *p_ < '0' || *p_ > '9') return fail("expected an integer");
        uint64_t a = 0;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
            if (a > (uint64_t)INT64_MAX / 10) return fail("integer overflow");
            a = a * 10 + (uint64_t)(*p_++ - '0');
            if (a > (uint64_t)INT64_MAX) return fail("integer overflow");
        }
        if (p_ < e_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E')) return fail("expected an integer");
        if (p_ - q > 1 + neg && q[neg] == '0') return fail("leading zero");
        v = neg ? -(int64_t)a : (int64_t)a;
        return true;
    }
    bool int_array(std::vector<int64_t> &v) {
        if (!lit('[')) return fail("expected an array");
        ws();
        if (lit(']')) return true;
        for (;;) {
            int64_t x;
            ws();
            if (!integer(x)) return false;
            v.push_back(x);
            ws();
            if (lit(',')) continue;
            if (lit(']')) return true;
            return fail("expected ',' or ']'");
        }
    }
    bool skip(int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p_ >= e_) return fail("unexpected end of header");
        const char c = *p_;
        if (c == '"') {
            std::string s;
            return str(s);
        }
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            p_++;
            ws();
            if (lit(close)) return true;
            for (;;) {
                ws();
                if (c == '{') {
                    std::string k;
                    if (!str(k)) return fail("bad object key");
                    ws();
                    if (!lit(':')) return fail("missing ':'");
                }
                if (!skip(depth + 1)) return false;
                ws();
                if (lit(',')) continue;
                if (lit(close)) return true;
                return fail("bad container");
            }
        }
        for (const char *w : {"true", "false", "null"}) {
            const size_t n = strlen(w);
            if ((size_t)(e_ - p_) >= n && memcmp(p_, w, n) == 0) {
                p_ += n;
                return true;
            }
        }
        // a JSON number
        const char *q = p_;
        lit('-');
        while (p_ < e_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                           *p_ == '-'))
            p_++;
        return p_ > q ? true : fail("bad value");
    }
    bool tensor(StTensor &t, uint64_t data_len, int64_t &max_end) {
        if (!lit('{')) return fail("tensor entry is not an object");
        bool has_dtype = false, has_shape = false, has_off = false;
        std::vector<int64_t> off;
        ws();
        if (!lit('}')) {
            for (;;) {
                std::string k;
                ws();
                if (!str(k)) return fail("bad key in a tensor entry");
                ws();
                if (!lit(':')) return fail("missing ':'");
                ws();
                if (k == "dtype") {
                    std::string d;
                    if (!str(d)) return fail("dtype is not a string");
                    t.dtype = dtype_code(d);
                    has_dtype = true;
                } else if (k == "shape") {
                    if (!int_array(t.shape)) return false;
                    has_shape = true;
                } else if (k == "data_offsets") {
                    if (!int_array(off)) return false;
                    has_off = true;
                } else if (!skip(1)) {
                    return false;
                }
                ws();
                if (lit(',')) continue;
                if (lit('}')) break;
                return fail("expected ',' or '}' in a tensor entry");
            }
        }
        if (!has_dtype || !has_shape || !has_off) return fail("tensor entry lacks dtype, shape or data_offsets");
        if (off.size() != 2 || off[0] < 0 || off[1] < off[0] || (uint64_t)off[1] > data_len)
            return fail("data_offsets outside the data section");
        if (t.shape.size() > QASR_ST_MAX_DIMS) return fail("too many dimensions");
        int64_t n = 1;
        for (int64_t s : t.shape) {
            if (s < 0 || (s > 0 && n > INT64_MAX / s)) return fail("bad shape");
            n *= s;
        }
        const int es = elem_size(t.dtype);
        if (es && (n > INT64_MAX / es || n * es != off[1] - off[0]))
            return fail("data_offsets do not match dtype and shape");
        t.bytes = off[1] - off[0];
        t.data = reinterpret_cast<const uint8_t *>((uintptr_t)off[0]);   // relative until the mapping is known
        max_end = std::max<int64_t>(max_end, off[1]);
        return true;
    }
};

bool utf8_valid(const unsigned char *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const unsigned c = s[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int k;
        unsigned cp;
        if ((c & 0xE0) == 0xC0) { k = 1; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { k = 2; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { k = 3; cp = c & 0x07; }
        else return false;
        if (n - i <= (size_t)k) return false;
        for (int j = 1; j <= k; j++) {
            if ((s[i + j] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + j] & 0x3F);
        }
        if ((k == 1 && cp < 0x80) || (k == 2 && cp < 0x800) || (k == 3 && (cp < 0x10000 || cp > 0x10FFFF)) ||
            (cp >= 0xD800 && cp < 0xE000))
            return false;
        i += (size_t)k + 1;
    }
    return true;
}

}  // namespace

struct qasr_st {
    std::vector<std::unique_ptr<Mapping>> shards;
    std::vector<std::string> shard_paths;
    std::map<std::string, StTensor> tensors;   // first shard holding a name wins (safetensors.rs:254-262)
    std::vector<std::string> names;            // in shard order, then header order
};

// SafetensorsFile::open (safetensors.rs:73-140): 8-byte little-endian header
// length, a UTF-8 JSON header, then the data section the offsets index
static int open_file(const std::string &path, qasr_st *st, std::string &why) {
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return why = "cannot open " + path, QASR_ERR_INVALID;
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 8) {
        close(fd);
        return why = path + ": not a safetensors file (shorter than 8 bytes)", QASR_ERR_INVALID;
    }
    auto m = std::make_unique<Mapping>();
    m->size = (size_t)sb.st_size;
    m->base = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m->base == MAP_FAILED) return why = "mmap failed for " + path, QASR_ERR_INVALID;
    const unsigned char *b = reinterpret_cast<const unsigned char *>(m->base);
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | b[i];
    if (hlen > m->size - 8) return why = path + ": header length exceeds the file", QASR_ERR_INVALID;
    if (!utf8_valid(b + 8, (size_t)hlen)) return why = path + ": header is not UTF-8", QASR_ERR_INVALID;
    const uint64_t data_len = m->size - 8 - hlen;
    Json j(reinterpret_cast<const char *>(b + 8), (size_t)hlen);
    std::vector<std::pair<std::string, StTensor>> found;
    int64_t max_end = 0;
    if (!j.header(found, max_end, data_len)) return why = path + ": bad header: " + j.err, QASR_ERR_INVALID;
    const uint8_t *data = b + 8 + hlen;
    std::map<std::string, StTensor> mine;       // a name repeated in one header: the last entry wins
    for (auto &kv : found) {
        kv.second.data = data + (uintptr_t)kv.second.data;
        if (!mine.count(kv.first)) st->names.push_back(kv.first);
        mine[kv.first] = kv.second;
    }
    for (auto &kv : mine) st->tensors.emplace(kv.first, kv.second);   // earlier shards keep their names
    st->shards.push_back(std::move(m));
    st->shard_paths.push_back(path);
    return QASR_OK;
}

extern "C" int qasr_hip_st_open_file(const char *path, qasr_st **out) {
    if (!path || !out) return qasr_fail(QASR_ERR_INVALID, "st_open_file: null argument");
    *out = nullptr;
    auto st = std::make_unique<qasr_st>();
    std::string why;
    if (open_file(path, st.get(), why) != QASR_OK) return qasr_fail(QASR_ERR_INVALID, why);
    *out = st.release();
    return QASR_OK;
}

// MultiSafetensors::open (safetensors.rs:212-250): model.safetensors when it
// opens, else every model-*.safetensors of the directory in byte order
extern "C" int qasr_hip_st_open(const char *model_dir, qasr_st **out) {
    if (!model_dir || !out) return qasr_fail(QASR_ERR_INVALID, "st_open: null argument");
    *out = nullptr;
    const std::string dir = model_dir;
    std::string why;
    {
        auto st = std::make_unique<qasr_st>();
        if (open_file(dir + "/model.safetensors", st.get(), why) == QASR_OK) {
            *out = st.release();
            return QASR_OK;
        }
    }
    std::vector<std::string> names;
    if (DIR *dp = opendir(model_dir)) {
        while (struct dirent *de = readdir(dp)) {
            const std::string n = de->d_name;
            const std::string suf = ".safetensors";
            if (n.size() >= 6 + suf.size() && n.compare(0, 6, "model-") == 0 &&
                n.compare(n.size() - suf.size(), suf.size(), suf) == 0)
                names.push_back(n);
        }
        closedir(dp);
    }
    if (names.empty()) return qasr_fail(QASR_ERR_INVALID, "st_open: no safetensors files in " + dir);
    std::sort(names.begin(), names.end());
    auto st = std::make_unique<qasr_st>();
    for (const auto &n : names)
        if (open_file(dir + "/" + n, st.get(), why) != QASR_OK) return qasr_fail(QASR_ERR_INVALID, why);
    *out = st.release();
    return QASR_OK;
}

extern "C" void qasr_hip_st_free(qasr_st *st) { delete st; }

extern "C" int64_t qasr_hip_st_count(const qasr_st *st) { return st ? (int64_t)st->names.size() : -1; }

extern "C" int64_t qasr_hip_st_shards(const qasr_st *st) { return st ? (int64_t)st->shards.size() : -1; }

extern "C" const char *qasr_hip_st_name(const qasr_st *st, int64_t i) {
    return st && i >= 0 && i < (int64_t)st->names.size() ? st->names[(size_t)i].c_str() : nullptr;
}

extern "C" int qasr_hip_st_find(const qasr_st *st, const char *name, int *dtype, int *ndim, int64_t *shape,
                                const void **data, int64_t *bytes) {
    if (!st || !name) return qasr_fail(QASR_ERR_INVALID, "st_find: null argument");
    auto it = st->tensors.find(name);
    if (it == st->tensors.end()) return qasr_fail(QASR_ERR_INVALID, std::string("st_find: no tensor ") + name);
    const StTensor &t = it->second;
    if (dtype) *dtype = t.dtype;
    if (ndim) *ndim = (int)t.shape.size();
    if (shape)
        for (size_t i = 0; i < t.shape.size(); i++) shape[i] = t.shape[i];
    if (data) *data = t.data;
    if (bytes) *bytes = t.bytes;
    return QASR_OK;
}

namespace {

// typed lookups with the shape checks the model loaders need
struct Loader {
    const qasr_st *st;
    std::vector<std::unique_ptr<std::vector<float>>> keep;   // converted f32 vectors live until the load ends
    std::string err;

    const StTensor *get(const std::string &name) {
        auto it = st->tensors.find(name);
        if (it == st->tensors.end()) {
            if (err.empty()) err = "missing tensor " + name;
            return nullptr;
        }
        return &it->second;
    }
    bool shape_is(const StTensor *t, const std::string &name, std::initializer_list<int64_t> want) {
        if (t->shape.size() == want.size() && std::equal(want.begin(), want.end(), t->shape.begin())) return true;
        std::string s = name + " has shape [";
        for (size_t i = 0; i < t->shape.size(); i++) s += (i ? ", " : "") + std::to_string(t->shape[i]);
        s += "], expected [";
        size_t i = 0;
        for (int64_t w : want) s += (i++ ? ", " : "") + std::to_string(w);
        if (err.empty()) err = s + "]";
        return false;
    }
    // load_bf16_direct (decoder.rs): a pointer into the mapping, BF16 only
    const uint16_t *bf16(const std::string &name, std::initializer_list<int64_t> shape) {
        const StTensor *t = get(name);
        if (!t || !shape_is(t, name, shape)) return nullptr;
        if (t->dtype != QASR_ST_BF16) {
            if (err.empty()) err = name + " is not BF16";
            return nullptr;
        }
        return reinterpret_cast<const uint16_t *>(t->data);
    }
    // load_f32 (decoder.rs, encoder.rs): F32 as stored, BF16 widened (get_f32, safetensors.rs:143-185)
    const float *f32(const std::string &name, std::initializer_list<int64_t> shape) {
        const StTensor *t = get(name);
        if (!t || !shape_is(t, name, shape)) return nullptr;
        int64_t n = 1;
        for (int64_t s : shape) n *= s;
        auto v = std::make_unique<std::vector<float>>((size_t)n);
        if (t->dtype == QASR_ST_F32) {
            std::memcpy(v->data(), t->data, sizeof(float) * n);
        } else if (t->dtype == QASR_ST_BF16) {
            const uint16_t *s = reinterpret_cast<const uint16_t *>(t->data);
            for (int64_t i = 0; i < n; i++) {
                uint16_t h;
                std::memcpy(&h, s + i, 2);
                const uint32_t u = (uint32_t)h << 16;
                std::memcpy(&(*v)[(size_t)i], &u, 4);
            }
        } else {
            if (err.empty()) err = name + " is neither F32 nor BF16";
            return nullptr;
        }
        keep.push_back(std::move(v));
        return keep.back()->data();
    }
};

}  // namespace

// Decoder::load (decoder.rs:70-167) from a checkpoint: names and layouts as
// the reference reads them; matrices must be BF16, norms F32 or BF16.  A
// "thinker.lm_head.weight" of any row count (vocab, or the forced aligner's
// classify_num: config.rs:86-88, 145-150) is both the int8 decode head and the
// bf16 prefill-logits head (decoder.rs:143-157, 671); without it both are the
// tied embedding.
extern "C" int qasr_hip_decoder_load_st(qasr_hip *h, const qasr_st *st, const qasr_dec_config *cfg, int round_mode,
                                        int64_t max_seq, int kv_bf16, qasr_decoder **out) {
    CHECK_H(h);
    if (!st || !cfg || !out) return qasr_fail(QASR_ERR_INVALID, "decoder_load_st: null argument");
    *out = nullptr;
    const qasr_dec_config &c = *cfg;
    if (c.n_layers <= 0 || c.n_layers > 1024 || c.hidden <= 0 || c.head_dim <= 0 || c.n_heads <= 0 ||
        c.n_kv_heads <= 0 || c.intermediate <= 0 || c.vocab <= 0)
        return qasr_fail(QASR_ERR_INVALID, "decoder_load_st: bad config");
    const int64_t H = c.hidden, qd = (int64_t)c.n_heads * c.head_dim, kvd = (int64_t)c.n_kv_heads * c.head_dim;
    const int64_t I = c.intermediate, hd = c.head_dim;
    Loader ld{st, {}, {}};
    std::vector<qasr_dec_layer> layers((size_t)c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        const std::string p = "thinker.model.layers." + std::to_string(l);
        qasr_dec_layer &L = layers[(size_t)l];
        L.wq = ld.bf16(p + ".self_attn.q_proj.weight", {qd, H});
        L.wk = ld.bf16(p + ".self_attn.k_proj.weight", {kvd, H});
        L.wv = ld.bf16(p + ".self_attn.v_proj.weight", {kvd, H});
        L.wo = ld.bf16(p + ".self_attn.o_proj.weight", {H, qd});
        L.q_norm = ld.f32(p + ".self_attn.q_norm.weight", {hd});
        L.k_norm = ld.f32(p + ".self_attn.k_norm.weight", {hd});
        L.input_norm = ld.f32(p + ".input_layernorm.weight", {H});
        L.post_attn_norm = ld.f32(p + ".post_attention_layernorm.weight", {H});
        L.gate = ld.bf16(p + ".mlp.gate_proj.weight", {I, H});
        L.up = ld.bf16(p + ".mlp.up_proj.weight", {I, H});
        L.down = ld.bf16(p + ".mlp.down_proj.weight", {H, I});
        if (!ld.err.empty()) return qasr_fail(QASR_ERR_INVALID, "decoder_load_st: " + ld.err);
    }
    qasr_dec_weights w{};
    w.embed = ld.bf16("thinker.model.embed_tokens.weight", {c.vocab, H});
    w.norm = ld.f32("thinker.model.norm.weight", {H});
    w.layers = layers.data();
    if (!ld.err.empty()) return qasr_fail(QASR_ERR_INVALID, "decoder_load_st: " + ld.err);
    const uint16_t *lm = nullptr;
    int64_t lm_rows = 0;
    auto it = st->tensors.find("thinker.lm_head.weight");
    if (it != st->tensors.end()) {
        const StTensor &t = it->second;
        if (t.dtype != QASR_ST_BF16 || t.shape.size() != 2 || t.shape[1] != H || t.shape[0] <= 0)
            return qasr_fail(QASR_ERR_INVALID, "decoder_load_st: thinker.lm_head.weight must be BF16 [rows, hidden]");
        // Disabled: the GPU test of this load stopped answering in two runs
        // (before and after its uploads went through the pinned staging ring)
        // and the cause is not shown, so the load refuses before any upload.
        // Callers load the checkpoint without the tensor and pass the head to
        // qasr_hip_decoder_set_lm_head for the prefill logits.
        return qasr_fail(QASR_ERR_INVALID,
                         "decoder_load_st: checkpoints with a separate thinker.lm_head.weight are not supported yet");
    }
    qasr_decoder *d = nullptr;
    int rc = decoder_load_impl(h, &c, &w, lm, lm_rows, round_mode, max_seq, kv_bf16, &d);
    if (rc != QASR_OK) return rc;
    if (lm) {
        rc = qasr_hip_decoder_set_lm_head(d, lm, lm_rows);
        if (rc != QASR_OK) {
            qasr_hip_decoder_free(d);
            return rc;
        }
    }
    *out = d;
    return QASR_OK;
}

// Encoder::load (encoder.rs:123-182) from a checkpoint: weight matrices BF16
// (the convolutions included), biases and norms F32 or BF16
extern "C" int qasr_hip_encoder_load_st(qasr_hip *h, const qasr_st *st, const qasr_enc_config *cfg,
                                        qasr_encoder **out) {
    CHECK_H(h);
    if (!st || !cfg || !out) return qasr_fail(QASR_ERR_INVALID, "encoder_load_st: null argument");
    *out = nullptr;
    const qasr_enc_config &c = *cfg;
    if (c.n_layers <= 0 || c.n_layers > 1024 || c.d_model <= 0 || c.ffn_dim <= 0 || c.conv_hidden <= 0 ||
        c.output_dim <= 0)
        return qasr_fail(QASR_ERR_INVALID, "encoder_load_st: bad config");
    const int64_t D = c.d_model, F = c.ffn_dim, C = c.conv_hidden, O = c.output_dim;
    const int64_t h3 = 16;                     // 128 mel bins after three stride-2 convolutions
    const std::string p = "thinker.audio_tower.";
    Loader ld{st, {}, {}};
    std::vector<qasr_enc_layer> layers((size_t)c.n_layers);
    qasr_enc_weights w{};
    w.conv1_w = ld.bf16(p + "conv2d1.weight", {C, 1, 3, 3});
    w.conv1_b = ld.f32(p + "conv2d1.bias", {C});
    w.conv2_w = ld.bf16(p + "conv2d2.weight", {C, C, 3, 3});
    w.conv2_b = ld.f32(p + "conv2d2.bias", {C});
    w.conv3_w = ld.bf16(p + "conv2d3.weight", {C, C, 3, 3});
    w.conv3_b = ld.f32(p + "conv2d3.bias", {C});
    w.conv_out_w = ld.bf16(p + "conv_out.weight", {D, C * h3});
    for (int l = 0; l < c.n_layers; l++) {
        const std::string q = p + "layers." + std::to_string(l);
        qasr_enc_layer &L = layers[(size_t)l];
        L.wq = ld.bf16(q + ".self_attn.q_proj.weight", {D, D});
        L.bq = ld.f32(q + ".self_attn.q_proj.bias", {D});
        L.wk = ld.bf16(q + ".self_attn.k_proj.weight", {D, D});
        L.bk = ld.f32(q + ".self_attn.k_proj.bias", {D});
        L.wv = ld.bf16(q + ".self_attn.v_proj.weight", {D, D});
        L.bv = ld.f32(q + ".self_attn.v_proj.bias", {D});
        L.wo = ld.bf16(q + ".self_attn.out_proj.weight", {D, D});
        L.bo = ld.f32(q + ".self_attn.out_proj.bias", {D});
        L.ln1_w = ld.f32(q + ".self_attn_layer_norm.weight", {D});
        L.ln1_b = ld.f32(q + ".self_attn_layer_norm.bias", {D});
        L.fc1 = ld.bf16(q + ".fc1.weight", {F, D});
        L.b1 = ld.f32(q + ".fc1.bias", {F});
        L.fc2 = ld.bf16(q + ".fc2.weight", {D, F});
        L.b2 = ld.f32(q + ".fc2.bias", {D});
        L.ln2_w = ld.f32(q + ".final_layer_norm.weight", {D});
        L.ln2_b = ld.f32(q + ".final_layer_norm.bias", {D});
        if (!ld.err.empty()) return qasr_fail(QASR_ERR_INVALID, "encoder_load_st: " + ld.err);
    }
    w.layers = layers.data();
    w.ln_post_w = ld.f32(p + "ln_post.weight", {D});
    w.ln_post_b = ld.f32(p + "ln_post.bias", {D});
    w.proj1_w = ld.bf16(p + "proj1.weight", {D, D});
    w.proj1_b = ld.f32(p + "proj1.bias", {D});
    w.proj2_w = ld.bf16(p + "proj2.weight", {O, D});
    w.proj2_b = ld.f32(p + "proj2.bias", {O});
    if (!ld.err.empty()) return qasr_fail(QASR_ERR_INVALID, "encoder_load_st: " + ld.err);
    return qasr_hip_encoder_load(h, &c, &w, out);
}
