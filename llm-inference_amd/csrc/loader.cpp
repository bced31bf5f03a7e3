// Checkpoint loading for the gfx950 build: config.json / generation_config.json and the
// safetensors shards of a model directory.
//
// The on-disk rules are the reference's (src/loader.cu:105-419): BF16 tensors only, shapes
// implied by config.json, data offsets 16-byte aligned, every tensor in the files used except a
// tied lm_head, lm_head = embedding when tie_word_embeddings. The design is this file's own:
//   1. config.json is read through a key table (JSON type and Config field per key);
//   2. every shard header is validated once into a manifest of tensor entries (name -> shard,
//      dtype, dims, byte range), rejecting malformed numbers before any cast;
//   3. the tensors the engine needs form a schema generated from the Config (name, dims, the
//      Weights/LayerWeights slot it fills), bound against the manifest in one pass;
//   4. only then is device memory touched: ONE allocation receives the schema's tensors, each
//      on a 256-byte boundary in schema order (the layout synth_weights produces), copied from
//      the memory-mapped shards.
// So every format or shape error is reported before any HIP call.
#include <dirent.h>
#include <fcntl.h>
#include <inttypes.h>
#include <math.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "errors.h"
#include "llm_amd/forward.h"

// ------------------------------------------------------------------------------------------
// JSON
// ------------------------------------------------------------------------------------------

namespace {

struct JVal {
    enum Type { NUL, BOOL, NUM, STR, ARR, OBJ } type = NUL;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;

    const JVal *get(const char *key) const {
        if (type != OBJ) return nullptr;
        for (const auto &kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonParser {
  public:
    JsonParser(const char *p, size_t n) : p_(p), end_(p + n) {}

    bool parse(JVal *out) {
        skip();
        if (!value(out, 0)) return false;
        skip();
        return p_ == end_;
    }

  private:
    const char *p_, *end_;

    void skip() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool lit(const char *s) {
        size_t n = strlen(s);
        if ((size_t)(end_ - p_) < n || memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void put_utf8(std::string *s, uint32_t cp) {
        if (cp < 0x80) {
            s->push_back((char)cp);
        } else if (cp < 0x800) {
            s->push_back((char)(0xC0 | (cp >> 6)));
            s->push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            s->push_back((char)(0xE0 | (cp >> 12)));
            s->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            s->push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            s->push_back((char)(0xF0 | (cp >> 18)));
            s->push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            s->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            s->push_back((char)(0x80 | (cp & 0x3F)));
        }
    }
    bool hex4(uint32_t *v) {
        if (end_ - p_ < 4) return false;
        *v = 0;
        for (int i = 0; i < 4; i++) {
            char c = *p_++;
            *v <<= 4;
            if (c >= '0' && c <= '9') *v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') *v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') *v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string *s) {
        if (p_ >= end_ || *p_ != '"') return false;
        p_++;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if ((unsigned char)c < 0x20) return false;
            if (c != '\\') {
                s->push_back(c);
                continue;
            }
            if (p_ >= end_) return false;
            c = *p_++;
            switch (c) {
            case '"': s->push_back('"'); break;
            case '\\': s->push_back('\\'); break;
            case '/': s->push_back('/'); break;
            case 'b': s->push_back('\b'); break;
            case 'f': s->push_back('\f'); break;
            case 'n': s->push_back('\n'); break;
            case 'r': s->push_back('\r'); break;
            case 't': s->push_back('\t'); break;
            case 'u': {
                uint32_t cp;
                if (!hex4(&cp)) return false;
                if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                    uint32_t lo;
                    if (!lit("\\u") || !hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                put_utf8(s, cp);
                break;
            }
            default: return false;
            }
        }
        if (p_ >= end_) return false;
        p_++;
        return true;
    }
    bool number(double *v) {
        const char *start = p_;
        if (p_ < end_ && *p_ == '-') p_++;
        if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return false;
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' ||
                             *p_ == 'E' || *p_ == '+' || *p_ == '-'))
            p_++;
        std::string tok(start, p_);
        char *e = nullptr;
        *v = strtod(tok.c_str(), &e);
        return e && *e == 0;
    }
    bool value(JVal *v, int depth) {
        if (depth > 64 || p_ >= end_) return false;
        char c = *p_;
        if (c == '{') {
            v->type = JVal::OBJ;
            p_++;
            skip();
            if (p_ < end_ && *p_ == '}') {
                p_++;
                return true;
            }
            for (;;) {
                skip();
                std::string key;
                if (!string(&key)) return false;
                skip();
                if (p_ >= end_ || *p_ != ':') return false;
                p_++;
                skip();
                JVal child;
                if (!value(&child, depth + 1)) return false;
                v->obj.emplace_back(std::move(key), std::move(child));
                skip();
                if (p_ < end_ && *p_ == ',') {
                    p_++;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    p_++;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            v->type = JVal::ARR;
            p_++;
            skip();
            if (p_ < end_ && *p_ == ']') {
                p_++;
                return true;
            }
            for (;;) {
                skip();
                JVal child;
                if (!value(&child, depth + 1)) return false;
                v->arr.push_back(std::move(child));
                skip();
                if (p_ < end_ && *p_ == ',') {
                    p_++;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    p_++;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            v->type = JVal::STR;
            return string(&v->str);
        }
        if (lit("true")) {
            v->type = JVal::BOOL;
            v->b = true;
            return true;
        }
        if (lit("false")) {
            v->type = JVal::BOOL;
            return true;
        }
        if (lit("null")) {
            v->type = JVal::NUL;
            return true;
        }
        v->type = JVal::NUM;
        return number(&v->num);
    }
};

bool read_text_file(const std::string &path, std::string *text) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) return llm_fail("loader: cannot open %s", path.c_str());
    fseek(f, 0, SEEK_END);
    long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    text->resize(size > 0 ? (size_t)size : 0);
    bool ok = size >= 0 && fread(&(*text)[0], 1, text->size(), f) == text->size();
    fclose(f);
    if (!ok) return llm_fail("loader: cannot read %s", path.c_str());
    return true;
}

bool parse_json_file(const std::string &path, JVal *root) {
    std::string text;
    if (!read_text_file(path, &text)) return false;
    JsonParser p(text.data(), text.size());
    if (!p.parse(root)) return llm_fail("loader: cannot parse %s", path.c_str());
    return true;
}

// A JSON number that is an exact non-negative integer no larger than `max` (safetensors
// offsets and dims, config sizes); anything else is rejected before it is cast.
bool json_uint(const JVal *v, double max, uint64_t *out) {
    if (!v || v->type != JVal::NUM) return false;
    const double d = v->num;
    if (!(d >= 0.0) || d > max || floor(d) != d) return false;
    *out = (uint64_t)d;
    return true;
}

}  // namespace

// ------------------------------------------------------------------------------------------
// config.json and generation_config.json
// ------------------------------------------------------------------------------------------

namespace {

enum KeyKind { KEY_INT, KEY_FLOAT, KEY_BOOL };

struct ConfigKey {
    const char *key;
    KeyKind kind;
    size_t field;  // offset of the Config member
};

// config.json entries the engine reads, in the order they are checked.
const ConfigKey kConfigKeys[] = {
    {"hidden_size", KEY_INT, offsetof(Config, hidden_size)},
    {"intermediate_size", KEY_INT, offsetof(Config, intermediate_size)},
    {"num_hidden_layers", KEY_INT, offsetof(Config, n_layers)},
    {"num_attention_heads", KEY_INT, offsetof(Config, n_heads)},
    {"num_key_value_heads", KEY_INT, offsetof(Config, n_kv_heads)},
    {"head_dim", KEY_INT, offsetof(Config, head_dim)},
    {"vocab_size", KEY_INT, offsetof(Config, vocab_size)},
    {"max_position_embeddings", KEY_INT, offsetof(Config, max_seq_len)},
    {"rms_norm_eps", KEY_FLOAT, offsetof(Config, rms_norm_eps)},
    {"rope_theta", KEY_FLOAT, offsetof(Config, rope_theta)},
    {"tie_word_embeddings", KEY_BOOL, offsetof(Config, tie_word_embeddings)},
};

bool read_config_key(const JVal &root, const ConfigKey &k, Config *cfg) {
    const JVal *v = root.get(k.key);
    char *field = (char *)cfg + k.field;
    switch (k.kind) {
    case KEY_BOOL:
        if (!v || v->type != JVal::BOOL)
            return llm_fail("loader: config.json has no bool \"%s\"", k.key);
        *(int *)field = v->b ? 1 : 0;
        return true;
    case KEY_FLOAT:
        if (!v || v->type != JVal::NUM)
            return llm_fail("loader: config.json has no number \"%s\"", k.key);
        *(float *)field = (float)v->num;
        return true;
    case KEY_INT: {
        if (!v || v->type != JVal::NUM)
            return llm_fail("loader: config.json has no number \"%s\"", k.key);
        uint64_t u;
        if (!json_uint(v, 2147483647.0, &u))
            return llm_fail("loader: config.json: \"%s\" must be a non-negative integer", k.key);
        *(int *)field = (int)u;
        return true;
    }
    }
    return false;
}

// eos_token_id: one id or a list of at most MAX_EOS ids.
bool read_eos(const char *model_dir, Config *cfg) {
    const std::string path = std::string(model_dir) + "/generation_config.json";
    JVal root;
    if (!parse_json_file(path, &root)) return false;
    const JVal *eos = root.get("eos_token_id");
    std::vector<const JVal *> ids;
    if (eos && eos->type == JVal::NUM) ids.push_back(eos);
    if (eos && eos->type == JVal::ARR)
        for (const JVal &id : eos->arr) ids.push_back(&id);
    if (ids.empty()) return llm_fail("loader: %s has no \"eos_token_id\"", path.c_str());
    if (ids.size() > MAX_EOS) return llm_fail("loader: %s: bad \"eos_token_id\"", path.c_str());
    cfg->n_eos = 0;
    for (const JVal *id : ids) {
        uint64_t u;
        if (!json_uint(id, 2147483647.0, &u))
            return llm_fail("loader: %s: bad \"eos_token_id\"", path.c_str());
        cfg->eos_ids[cfg->n_eos++] = (int)u;
    }
    return true;
}

}  // namespace

extern "C" void load_config(const char *model_dir, Config *cfg) {
    memset(cfg, 0, sizeof *cfg);
    JVal root;
    if (!parse_json_file(std::string(model_dir) + "/config.json", &root)) return;
    for (const ConfigKey &k : kConfigKeys)
        if (!read_config_key(root, k, cfg)) return;
    if (cfg->n_kv_heads <= 0 || cfg->n_heads % cfg->n_kv_heads != 0) {
        llm_fail("loader: num_attention_heads must be a multiple of num_key_value_heads");
        return;
    }
    read_eos(model_dir, cfg);
}

// ------------------------------------------------------------------------------------------
// safetensors: [u64 little-endian header length N][N bytes of JSON header][data section];
// header entries {"dtype", "shape", "data_offsets": [begin, end]} relative to the data section.
// ------------------------------------------------------------------------------------------

namespace {

struct MappedFile {
    std::string path;
    const char *bytes = nullptr;  // the whole file, read-only
    size_t size = 0;
    const char *data = nullptr;   // start of the data section
    size_t data_bytes = 0;
};

struct Entry {
    std::string name, dtype;
    int shard = 0;
    std::vector<uint64_t> dims;
    uint64_t begin = 0, end = 0;
    bool used = false;
};

// Every tensor of every shard, validated when the headers are read.
struct Manifest {
    std::vector<MappedFile> files;
    std::vector<Entry> entries;
    std::unordered_map<std::string, size_t> index;

    ~Manifest() {
        for (MappedFile &f : files)
            if (f.bytes) munmap((void *)f.bytes, f.size);
    }
    const Entry *find(const std::string &name) const {
        auto it = index.find(name);
        return it == index.end() ? nullptr : &entries[it->second];
    }
};

bool map_file(const std::string &path, MappedFile *f) {
    f->path = path;
    const int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) return llm_fail("loader: cannot open %s", path.c_str());
    struct stat st;
    const bool stat_ok = fstat(fd, &st) == 0;
    if (!stat_ok || st.st_size < 8) {
        close(fd);
        return stat_ok ? llm_fail("loader: %s: too small to be a safetensors file", path.c_str())
                       : llm_fail("loader: cannot stat %s", path.c_str());
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return llm_fail("loader: cannot mmap %s", path.c_str());
    f->bytes = (const char *)m;
    f->size = (size_t)st.st_size;
    return true;
}

// One entry of a shard header: every number a non-negative integer, the byte range inside the
// data section and 16-byte aligned; for BF16, the range holds exactly the shape's elements.
bool read_entry(const MappedFile &f, int shard, const std::string &name, const JVal &e,
                Entry *out) {
    const char *p = f.path.c_str(), *n = name.c_str();
    const JVal *dtype = e.get("dtype"), *shape = e.get("shape"), *offs = e.get("data_offsets");
    if (!dtype || dtype->type != JVal::STR)
        return llm_fail("loader: %s: tensor %s has no dtype", p, n);
    if (!shape || shape->type != JVal::ARR)
        return llm_fail("loader: %s: tensor %s has no shape", p, n);
    if (!offs || offs->type != JVal::ARR || offs->arr.size() != 2)
        return llm_fail("loader: %s: tensor %s: data_offsets must be [begin, end]", p, n);
    out->name = name;
    out->dtype = dtype->str;
    out->shard = shard;
    uint64_t numel = 1;
    for (const JVal &d : shape->arr) {
        uint64_t v;
        if (!json_uint(&d, 4294967295.0, &v))
            return llm_fail("loader: %s: tensor %s: dims must be non-negative integers", p, n);
        out->dims.push_back(v);
        numel *= v;
    }
    if (!json_uint(&offs->arr[0], 9007199254740992.0, &out->begin) ||
        !json_uint(&offs->arr[1], 9007199254740992.0, &out->end))
        return llm_fail("loader: %s: tensor %s: data_offsets must be non-negative integers", p, n);
    if (out->end < out->begin || out->end > f.data_bytes)
        return llm_fail("loader: %s: tensor %s: data_offsets [%" PRIu64 ", %" PRIu64
                        ") outside the %zu-byte data section",
                        p, n, out->begin, out->end, f.data_bytes);
    if (out->begin % 16 != 0)
        return llm_fail("loader: %s: tensor %s: offset %" PRIu64 " is not 16-byte aligned", p, n,
                        out->begin);
    if (out->dtype == "BF16" && out->end - out->begin != numel * 2)
        return llm_fail("loader: %s: tensor %s: %" PRIu64 " bytes for %" PRIu64 " bf16 elements",
                        p, n, out->end - out->begin, numel);
    return true;
}

bool read_shard(MappedFile *f, int shard, Manifest *m) {
    uint64_t header_len;
    memcpy(&header_len, f->bytes, 8);
    if (header_len > f->size - 8) return llm_fail("loader: %s: bad header length", f->path.c_str());
    JVal header;
    JsonParser parser(f->bytes + 8, (size_t)header_len);
    if (!parser.parse(&header) || header.type != JVal::OBJ)
        return llm_fail("loader: %s: cannot parse header", f->path.c_str());
    f->data = f->bytes + 8 + header_len;
    f->data_bytes = f->size - 8 - (size_t)header_len;
    for (const auto &kv : header.obj) {
        if (kv.first == "__metadata__") continue;
        Entry e;
        if (!read_entry(*f, shard, kv.first, kv.second, &e)) return false;
        if (m->index.count(e.name))
            return llm_fail("loader: tensor %s appears in more than one place", e.name.c_str());
        m->index.emplace(e.name, m->entries.size());
        m->entries.push_back(std::move(e));
    }
    return true;
}

bool read_manifest(const char *model_dir, Manifest *m) {
    DIR *dir = opendir(model_dir);
    if (!dir) return llm_fail("loader: cannot open directory %s", model_dir);
    std::vector<std::string> names;
    for (struct dirent *e = readdir(dir); e; e = readdir(dir)) {
        const size_t len = strlen(e->d_name), ext = strlen(".safetensors");
        if (len > ext && strcmp(e->d_name + len - ext, ".safetensors") == 0)
            names.push_back(e->d_name);
    }
    closedir(dir);
    if (names.empty()) return llm_fail("loader: no .safetensors files in %s", model_dir);
    if (names.size() > MAX_SHARDS)
        return llm_fail("loader: %zu .safetensors files in %s (at most %d)", names.size(),
                        model_dir, MAX_SHARDS);
    std::sort(names.begin(), names.end());
    m->files.resize(names.size());
    for (size_t i = 0; i < names.size(); i++)
        if (!map_file(std::string(model_dir) + "/" + names[i], &m->files[i]) ||
            !read_shard(&m->files[i], (int)i, m))
            return false;
    return true;
}

// ---- the schema: the tensors the engine reads, generated from the Config

enum Dim { D_NONE, D_H, D_I, D_QD, D_KVD, D_HEAD, D_VOCAB };

struct LayerTensor {
    const char *suffix;  // after "model.layers.<l>."
    Dim rows, cols;      // cols D_NONE: a vector of `rows` elements
    const bf16 *LayerWeights::*slot;
};

const LayerTensor kLayerTensors[] = {
    {"input_layernorm.weight", D_H, D_NONE, &LayerWeights::attn_norm},
    {"self_attn.q_proj.weight", D_QD, D_H, &LayerWeights::wq},
    {"self_attn.k_proj.weight", D_KVD, D_H, &LayerWeights::wk},
    {"self_attn.v_proj.weight", D_KVD, D_H, &LayerWeights::wv},
    {"self_attn.q_norm.weight", D_HEAD, D_NONE, &LayerWeights::q_norm},
    {"self_attn.k_norm.weight", D_HEAD, D_NONE, &LayerWeights::k_norm},
    {"self_attn.o_proj.weight", D_H, D_QD, &LayerWeights::wo},
    {"post_attention_layernorm.weight", D_H, D_NONE, &LayerWeights::mlp_norm},
    {"mlp.gate_proj.weight", D_I, D_H, &LayerWeights::w_gate},
    {"mlp.up_proj.weight", D_I, D_H, &LayerWeights::w_up},
    {"mlp.down_proj.weight", D_H, D_I, &LayerWeights::w_down},
};

struct Want {
    std::string name;
    std::vector<uint64_t> dims;
    const bf16 **slot;
    const Entry *entry = nullptr;
    size_t dev_offset = 0;  // inside the one device allocation
};

uint64_t dim_size(const Config *c, Dim d) {
    switch (d) {
    case D_H: return (uint64_t)c->hidden_size;
    case D_I: return (uint64_t)c->intermediate_size;
    case D_QD: return (uint64_t)c->n_heads * c->head_dim;
    case D_KVD: return (uint64_t)c->n_kv_heads * c->head_dim;
    case D_HEAD: return (uint64_t)c->head_dim;
    case D_VOCAB: return (uint64_t)c->vocab_size;
    default: return 0;
    }
}

std::vector<Want> make_schema(const Config *c, Weights *w) {
    std::vector<Want> s;
    auto add = [&](std::string name, Dim rows, Dim cols, const bf16 **slot) {
        Want x;
        x.name = std::move(name);
        x.dims.push_back(dim_size(c, rows));
        if (cols != D_NONE) x.dims.push_back(dim_size(c, cols));
        x.slot = slot;
        s.push_back(std::move(x));
    };
    add("model.embed_tokens.weight", D_VOCAB, D_H, &w->embed);
    for (int l = 0; l < c->n_layers; l++)
        for (const LayerTensor &t : kLayerTensors)
            add("model.layers." + std::to_string(l) + "." + t.suffix, t.rows, t.cols,
                &(w->layers[l].*t.slot));
    add("model.norm.weight", D_H, D_NONE, &w->final_norm);
    if (!c->tie_word_embeddings) add("lm_head.weight", D_VOCAB, D_H, &w->lm_head);
    return s;
}

std::string dims_text(const std::vector<uint64_t> &d) {
    std::string s = "[";
    for (size_t i = 0; i < d.size(); i++) s += (i ? ", " : "") + std::to_string(d[i]);
    return s + "]";
}

// Each wanted tensor found, BF16, with the Config's shape; then nothing left over but a tied
// lm_head.
bool bind(std::vector<Want> &schema, Manifest &m, bool tied) {
    for (Want &x : schema) {
        const Entry *e = m.find(x.name);
        if (!e) return llm_fail("loader: tensor %s not found", x.name.c_str());
        if (e->dtype != "BF16")
            return llm_fail("loader: tensor %s is %s, only BF16 is supported", x.name.c_str(),
                            e->dtype.c_str());
        if (e->dims != x.dims)
            return llm_fail("loader: tensor %s has shape %s, config.json implies %s",
                            x.name.c_str(), dims_text(e->dims).c_str(), dims_text(x.dims).c_str());
        x.entry = e;
        m.entries[e - m.entries.data()].used = true;
    }
    int unused = 0;
    const char *first = nullptr;
    for (const Entry &e : m.entries)
        if (!e.used && !(tied && e.name == "lm_head.weight")) {
            if (!first) first = e.name.c_str();
            unused++;
        }
    if (unused)
        return llm_fail("loader: %d tensor(s) in the checkpoint are not read by the engine "
                        "(first: %s)",
                        unused, first);
    return true;
}

}  // namespace

extern "C" void free_weights(Weights *w) {
    for (int i = 0; i < w->n_buffers; i++)
        if (w->gpu_buffers[i]) HIP_OK(hipFree(w->gpu_buffers[i]));
    free(w->layers);
    free(w->tensors);
    memset(w, 0, sizeof *w);
}

extern "C" void load_weights(const char *model_dir, const Config *cfg, Weights *w) {
    memset(w, 0, sizeof *w);
    if (cfg->n_layers <= 0) {
        llm_fail("loader: num_hidden_layers %d must be positive", cfg->n_layers);
        return;
    }
    w->layers = (LayerWeights *)calloc((size_t)cfg->n_layers, sizeof(LayerWeights));
    if (!w->layers) {
        llm_fail("loader: out of memory");
        return;
    }
    Manifest m;
    std::vector<Want> schema = make_schema(cfg, w);
    if (!read_manifest(model_dir, &m) || !bind(schema, m, cfg->tie_word_embeddings != 0)) {
        free_weights(w);
        return;
    }
    size_t total = 0;
    for (Want &x : schema) {
        x.dev_offset = total;
        total += ((x.entry->end - x.entry->begin) + 255) & ~(size_t)255;
    }
    w->tensors = (TensorRef *)calloc(schema.size(), sizeof(TensorRef));
    char *base = nullptr;
    if (!w->tensors) {
        llm_fail("loader: out of memory");
        free_weights(w);
        return;
    }
    if (!HIP_OK(hipMalloc((void **)&base, total ? total : 256))) {
        free_weights(w);
        return;
    }
    w->gpu_buffers[0] = base;
    w->n_buffers = 1;
    w->gpu_bytes = total;
    for (size_t i = 0; i < schema.size(); i++) {
        const Want &x = schema[i];
        const Entry &e = *x.entry;
        const bf16 *dst = (const bf16 *)(base + x.dev_offset);
        if (!HIP_OK(hipMemcpy((void *)dst, m.files[e.shard].data + e.begin, e.end - e.begin,
                              hipMemcpyHostToDevice))) {
            free_weights(w);
            return;
        }
        *x.slot = dst;
        TensorRef *t = &w->tensors[i];
        snprintf(t->name, sizeof t->name, "%s", x.name.c_str());
        t->data = dst;
        t->numel = (e.end - e.begin) / 2;
    }
    w->n_tensors = (int)schema.size();
    if (cfg->tie_word_embeddings) w->lm_head = w->embed;
}

// Per tensor (ref/weight_checksums.py's contract, src/loader.cu:395-419 line format):
// "<name> <numel> <sum of the raw bf16 bits> <sum of bits * (index + 1)> <first value>", the
// sums exact modulo 2^64. The tensor is read back in bounded pieces.
extern "C" void print_weight_checksums(const Weights *w) {
    const size_t PIECE = (size_t)8 << 20;  // elements per read-back
    std::vector<uint16_t> buf;
    for (int i = 0; i < w->n_tensors; i++) {
        const TensorRef *t = &w->tensors[i];
        uint64_t sum = 0, weighted = 0;
        uint16_t first = 0;
        for (size_t at = 0; at < t->numel; at += PIECE) {
            const size_t n = std::min(PIECE, t->numel - at);
            buf.resize(n);
            if (!HIP_OK(hipMemcpy(buf.data(), t->data + at, n * 2, hipMemcpyDeviceToHost))) return;
            if (at == 0) first = buf[0];
            for (size_t j = 0; j < n; j++) {
                sum += buf[j];
                weighted += (uint64_t)(at + j + 1) * buf[j];
            }
        }
        uint32_t fbits = (uint32_t)first << 16;
        float fval;
        memcpy(&fval, &fbits, 4);
        printf("%s %zu %" PRIu64 " %" PRIu64 " %.6g\n", t->name, t->numel, sum, weighted, fval);
    }
    fflush(stdout);
}
