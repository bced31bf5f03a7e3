// Checkpoint loading for the gfx950 build: config.json / generation_config.json and
// safetensors shards (src/loader.cu:105-419 semantics: BF16 only, shapes implied by the config,
// 16-byte-aligned data offsets, every tensor in the files used, lm_head tied to the embedding
// when tie_word_embeddings). JSON is read by the small parser below.
#include <dirent.h>
#include <fcntl.h>
#include <inttypes.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <string>
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

bool json_number(const JVal &root, const char *key, double *v) {
    const JVal *item = root.get(key);
    if (!item || item->type != JVal::NUM)
        return llm_fail("loader: config.json has no number \"%s\"", key);
    *v = item->num;
    return true;
}

}  // namespace

// ------------------------------------------------------------------------------------------
// config (src/loader.cu:73-139)
// ------------------------------------------------------------------------------------------

static bool load_eos_ids(const char *model_dir, Config *cfg) {
    std::string path = std::string(model_dir) + "/generation_config.json";
    JVal root;
    if (!parse_json_file(path, &root)) return false;
    const JVal *eos = root.get("eos_token_id");
    cfg->n_eos = 0;
    if (eos && eos->type == JVal::NUM) {
        cfg->eos_ids[0] = (int)eos->num;
        cfg->n_eos = 1;
    } else if (eos && eos->type == JVal::ARR) {
        for (const JVal &id : eos->arr) {
            if (id.type != JVal::NUM || cfg->n_eos == MAX_EOS)
                return llm_fail("loader: %s: bad \"eos_token_id\"", path.c_str());
            cfg->eos_ids[cfg->n_eos++] = (int)id.num;
        }
    }
    if (cfg->n_eos == 0) return llm_fail("loader: %s has no \"eos_token_id\"", path.c_str());
    return true;
}

extern "C" void load_config(const char *model_dir, Config *cfg) {
    memset(cfg, 0, sizeof *cfg);
    std::string path = std::string(model_dir) + "/config.json";
    JVal root;
    if (!parse_json_file(path, &root)) return;
    const struct {
        const char *key;
        int *dst;
    } ints[] = {{"hidden_size", &cfg->hidden_size},
                {"intermediate_size", &cfg->intermediate_size},
                {"num_hidden_layers", &cfg->n_layers},
                {"num_attention_heads", &cfg->n_heads},
                {"num_key_value_heads", &cfg->n_kv_heads},
                {"head_dim", &cfg->head_dim},
                {"vocab_size", &cfg->vocab_size},
                {"max_position_embeddings", &cfg->max_seq_len}};
    double v;
    for (const auto &f : ints) {
        if (!json_number(root, f.key, &v)) return;
        *f.dst = (int)v;
    }
    if (!json_number(root, "rms_norm_eps", &v)) return;
    cfg->rms_norm_eps = (float)v;
    if (!json_number(root, "rope_theta", &v)) return;
    cfg->rope_theta = (float)v;
    const JVal *tie = root.get("tie_word_embeddings");
    if (!tie || tie->type != JVal::BOOL) {
        llm_fail("loader: config.json has no bool \"tie_word_embeddings\"");
        return;
    }
    cfg->tie_word_embeddings = tie->b ? 1 : 0;
    if (cfg->n_kv_heads <= 0 || cfg->n_heads % cfg->n_kv_heads != 0) {
        llm_fail("loader: num_attention_heads must be a multiple of num_key_value_heads");
        return;
    }
    load_eos_ids(model_dir, cfg);
}

// ------------------------------------------------------------------------------------------
// safetensors (src/loader.cu:141-380)
// ------------------------------------------------------------------------------------------

namespace {

struct Shard {
    std::string path;
    JVal header;
    char *gpu_data = nullptr;
    size_t data_bytes = 0;
};

// [u64 little-endian header length N][N bytes of JSON][data]; offsets are relative to the data.
bool load_shard(const std::string &path, Shard *shard) {
    shard->path = path;
    int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) return llm_fail("loader: cannot open %s", path.c_str());
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return llm_fail("loader: cannot stat %s", path.c_str());
    }
    const size_t file_size = (size_t)st.st_size;
    if (file_size < 8) {
        close(fd);
        return llm_fail("loader: %s: too small to be a safetensors file", path.c_str());
    }
    void *map = mmap(nullptr, file_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return llm_fail("loader: cannot mmap %s", path.c_str());
    const char *bytes = (const char *)map;
    uint64_t header_len;
    memcpy(&header_len, bytes, 8);
    bool ok = true;
    if (header_len > file_size - 8) {
        ok = llm_fail("loader: %s: bad header length", path.c_str());
    } else {
        JsonParser p(bytes + 8, (size_t)header_len);
        if (!p.parse(&shard->header) || shard->header.type != JVal::OBJ) {
            ok = llm_fail("loader: %s: cannot parse header", path.c_str());
        } else {
            shard->data_bytes = file_size - 8 - header_len;
            ok = HIP_OK(hipMalloc((void **)&shard->gpu_data, shard->data_bytes ? shard->data_bytes : 16)) &&
                 HIP_OK(hipMemcpy(shard->gpu_data, bytes + 8 + header_len, shard->data_bytes,
                                  hipMemcpyHostToDevice));
        }
    }
    munmap(map, file_size);
    return ok;
}

struct Loader {
    std::vector<Shard> shards;
    Weights *w = nullptr;
    int max_tensors = 0;

    const JVal *lookup(const char *name, const Shard **shard) const {
        for (const Shard &s : shards) {
            const JVal *e = s.header.get(name);
            if (e) {
                *shard = &s;
                return e;
            }
        }
        return nullptr;
    }

    const bf16 *find(const char *name, int n_dims, const int *shape) {
        const Shard *shard = nullptr;
        const JVal *e = lookup(name, &shard);
        if (!e) return llm_fail("loader: tensor %s not found", name), nullptr;
        const JVal *dtype = e->get("dtype");
        if (!dtype || dtype->type != JVal::STR || dtype->str != "BF16")
            return llm_fail("loader: %s: dtype is not BF16", name), nullptr;
        const JVal *dims = e->get("shape");
        if (!dims || dims->type != JVal::ARR || (int)dims->arr.size() != n_dims)
            return llm_fail("loader: %s: expected %d dims", name, n_dims), nullptr;
        size_t numel = 1;
        for (int d = 0; d < n_dims; d++) {
            const int got = (int)dims->arr[d].num;
            if (got != shape[d])
                return llm_fail("loader: %s: dim %d is %d, config.json implies %d", name, d, got,
                                shape[d]),
                       nullptr;
            numel *= (size_t)shape[d];
        }
        const JVal *off = e->get("data_offsets");
        if (!off || off->type != JVal::ARR || off->arr.size() != 2)
            return llm_fail("loader: %s: bad data_offsets", name), nullptr;
        const size_t begin = (size_t)off->arr[0].num, end = (size_t)off->arr[1].num;
        if (end > shard->data_bytes || end < begin || end - begin != numel * 2)
            return llm_fail("loader: %s: data_offsets do not match its shape", name), nullptr;
        if (begin % 16 != 0)
            return llm_fail("loader: %s: offset %zu is not 16-byte aligned", name, begin), nullptr;
        if (w->n_tensors == max_tensors)
            return llm_fail("loader: %s: loaded more tensors than the files contain", name), nullptr;
        const bf16 *data = (const bf16 *)(shard->gpu_data + begin);
        TensorRef *ref = &w->tensors[w->n_tensors++];
        snprintf(ref->name, sizeof ref->name, "%s", name);
        ref->data = data;
        ref->numel = numel;
        return data;
    }
};

bool ends_with(const std::string &s, const char *suffix) {
    size_t n = strlen(suffix);
    return s.size() >= n && s.compare(s.size() - n, n, suffix) == 0;
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
    Loader ld;
    ld.w = w;
    DIR *dir = opendir(model_dir);
    if (!dir) {
        llm_fail("loader: cannot open directory %s", model_dir);
        return;
    }
    std::vector<std::string> files;
    for (struct dirent *e = readdir(dir); e; e = readdir(dir))
        if (ends_with(e->d_name, ".safetensors")) files.push_back(e->d_name);
    closedir(dir);
    std::sort(files.begin(), files.end());
    if (files.empty()) {
        llm_fail("loader: no .safetensors files in %s", model_dir);
        return;
    }
    if (files.size() > MAX_SHARDS) {
        llm_fail("loader: more than %d .safetensors files in %s", MAX_SHARDS, model_dir);
        return;
    }
    ld.shards.resize(files.size());
    auto release = [&]() {
        for (Shard &s : ld.shards)
            if (s.gpu_data) (void)hipFree(s.gpu_data);
        free(w->tensors);
        free(w->layers);
        memset(w, 0, sizeof *w);
    };
    for (size_t i = 0; i < files.size(); i++)
        if (!load_shard(std::string(model_dir) + "/" + files[i], &ld.shards[i])) {
            release();
            return;
        }
    int in_files = 0;
    for (const Shard &s : ld.shards) {
        in_files += (int)s.header.obj.size();
        if (s.header.get("__metadata__")) in_files--;
    }
    w->tensors = (TensorRef *)calloc(in_files > 0 ? in_files : 1, sizeof(TensorRef));
    w->layers = (LayerWeights *)calloc(cfg->n_layers > 0 ? cfg->n_layers : 1, sizeof(LayerWeights));
    ld.max_tensors = in_files;
    const int H = cfg->hidden_size, D = cfg->head_dim, I = cfg->intermediate_size;
    const int q_dim = cfg->n_heads * D, kv_dim = cfg->n_kv_heads * D;
    auto vec = [&](const char *name, int n) { return ld.find(name, 1, &n); };
    auto mat = [&](const char *name, int r, int c) {
        int shape[2] = {r, c};
        return ld.find(name, 2, shape);
    };
    char name[96];
    auto lname = [&](int l, const char *suffix) {
        snprintf(name, sizeof name, "model.layers.%d.%s", l, suffix);
        return name;
    };
    w->embed = mat("model.embed_tokens.weight", cfg->vocab_size, H);
    for (int l = 0; l < cfg->n_layers && !llm_has_error(); l++) {
        LayerWeights *L = &w->layers[l];
        L->attn_norm = vec(lname(l, "input_layernorm.weight"), H);
        L->wq = mat(lname(l, "self_attn.q_proj.weight"), q_dim, H);
        L->wk = mat(lname(l, "self_attn.k_proj.weight"), kv_dim, H);
        L->wv = mat(lname(l, "self_attn.v_proj.weight"), kv_dim, H);
        L->q_norm = vec(lname(l, "self_attn.q_norm.weight"), D);
        L->k_norm = vec(lname(l, "self_attn.k_norm.weight"), D);
        L->wo = mat(lname(l, "self_attn.o_proj.weight"), H, q_dim);
        L->mlp_norm = vec(lname(l, "post_attention_layernorm.weight"), H);
        L->w_gate = mat(lname(l, "mlp.gate_proj.weight"), I, H);
        L->w_up = mat(lname(l, "mlp.up_proj.weight"), I, H);
        L->w_down = mat(lname(l, "mlp.down_proj.weight"), H, I);
    }
    if (!llm_has_error()) w->final_norm = vec("model.norm.weight", H);
    if (!llm_has_error())
        w->lm_head = cfg->tie_word_embeddings ? w->embed : mat("lm_head.weight", cfg->vocab_size, H);
    if (llm_has_error()) {
        release();
        return;
    }
    const Shard *unused_shard = nullptr;
    const int allowed = (cfg->tie_word_embeddings && ld.lookup("lm_head.weight", &unused_shard)) ? 1 : 0;
    const int unused = in_files - w->n_tensors;
    if (unused != allowed) {
        llm_fail("loader: %d tensors in the safetensors files are not used by the engine", unused);
        release();
        return;
    }
    for (size_t i = 0; i < ld.shards.size(); i++) {
        w->gpu_buffers[i] = ld.shards[i].gpu_data;
        w->gpu_bytes += ld.shards[i].data_bytes;
    }
    w->n_buffers = (int)ld.shards.size();
}

// src/loader.cu:395-419: per tensor, exact uint64 sums of the raw bits (plain and weighted by
// position + 1), read back from the device.
extern "C" void print_weight_checksums(const Weights *w) {
    for (int i = 0; i < w->n_tensors; i++) {
        const TensorRef *t = &w->tensors[i];
        std::vector<uint16_t> bits(t->numel);
        if (!HIP_OK(hipMemcpy(bits.data(), t->data, t->numel * 2, hipMemcpyDeviceToHost))) return;
        uint64_t sum = 0, weighted = 0;
        for (size_t j = 0; j < t->numel; j++) {
            sum += bits[j];
            weighted += (uint64_t)(j + 1) * bits[j];
        }
        uint32_t first_bits = (uint32_t)(t->numel ? bits[0] : 0) << 16;
        float first;
        memcpy(&first, &first_bits, 4);
        printf("%s %zu %" PRIu64 " %" PRIu64 " %.6g\n", t->name, t->numel, sum, weighted, first);
    }
    fflush(stdout);
}
