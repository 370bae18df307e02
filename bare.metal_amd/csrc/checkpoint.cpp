/* SPDX-License-Identifier: MPL-2.0
 *
 * checkpoint.cpp — Hugging Face checkpoint input for the engine: config.json
 * to bm_arch_t and safetensors tensors (F32 or BF16, one file or shards
 * listed by model.safetensors.index.json) into a model's weights.
 *
 * Reference behaviour followed:
 *   - config keys and defaults: reference src/baremetal/config.c:128-297
 *     (text_config section, GPT-2 style fallbacks, rope_scaling "llama3",
 *     RMSNorm iff rms_norm_eps is present, SwiGLU iff the activation names
 *     silu/swiglu, RoPE iff rope_theta is present, max_seq_len 2048 when
 *     max_position_embeddings is absent);
 *   - tensor names of the llama family and their grouping by matrix type:
 *     reference src/baremetal/config.c:13-31, checkpoint_st.c:430-691
 *     (a checkpoint without lm_head is tied);
 *   - shard discovery: index.json weight_map, else every *.safetensors file
 *     of the directory in name order (checkpoint_st.c:258-330).
 * BF16 projections stay bf16 on the host and are packed to Q8 on the device
 * from bf16 (the reference's bmt_quantize_q8_bf16, quant.c:62-71); other
 * bf16 tensors are widened exactly (bits << 16), as types.h:15-20 does.
 *
 * Host code only: no device calls here (bm_compile uploads).
 */
#include "bmk.h"
#include "baremetal.h"

#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

namespace {

/* ---- a small JSON reader (objects, arrays, strings, numbers, literals) ---- */

struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const char* key) const {
        if (kind != OBJ) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

struct JsonParser {
    const char* p;
    const char* end;
    std::string err;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool fail(const char* what) {
        if (err.empty()) err = what;
        return false;
    }
    bool string(std::string& out) {
        if (p >= end || *p != '"') return fail("expected a string");
        p++;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p >= end) return fail("bad escape");
            c = *p++;
            switch (c) {
                case 'n': out.push_back('\n'); break;
                case 't': out.push_back('\t'); break;
                case 'r': out.push_back('\r'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'u': {
                    if (end - p < 4) return fail("bad \\u escape");
                    unsigned v = (unsigned)strtoul(std::string(p, 4).c_str(), nullptr, 16);
                    p += 4;
                    /* names and keys here are ASCII; keep BMP code points as UTF-8 */
                    if (v < 0x80) out.push_back((char)v);
                    else if (v < 0x800) {
                        out.push_back((char)(0xC0 | (v >> 6)));
                        out.push_back((char)(0x80 | (v & 0x3F)));
                    } else {
                        out.push_back((char)(0xE0 | (v >> 12)));
                        out.push_back((char)(0x80 | ((v >> 6) & 0x3F)));
                        out.push_back((char)(0x80 | (v & 0x3F)));
                    }
                    break;
                }
                default: out.push_back(c); break;
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end");
        if (*p == '{') {
            p++;
            v.kind = Json::OBJ;
            ws();
            if (p < end && *p == '}') {
                p++;
                return true;
            }
            for (;;) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p >= end || *p != ':') return fail("expected ':'");
                p++;
                v.obj.emplace_back(std::move(key), Json());
                if (!value(v.obj.back().second, depth + 1)) return false;
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == '}') {
                    p++;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (*p == '[') {
            p++;
            v.kind = Json::ARR;
            ws();
            if (p < end && *p == ']') {
                p++;
                return true;
            }
            for (;;) {
                v.arr.emplace_back();
                if (!value(v.arr.back(), depth + 1)) return false;
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == ']') {
                    p++;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (*p == '"') {
            v.kind = Json::STR;
            return string(v.str);
        }
        if (end - p >= 4 && !strncmp(p, "true", 4)) {
            v.kind = Json::BOOL;
            v.b = true;
            p += 4;
            return true;
        }
        if (end - p >= 5 && !strncmp(p, "false", 5)) {
            v.kind = Json::BOOL;
            p += 5;
            return true;
        }
        if (end - p >= 4 && !strncmp(p, "null", 4)) {
            p += 4;
            return true;
        }
        /* number */
        std::string tok;
        while (p < end && (strchr("+-0123456789.eE", *p) != nullptr)) tok.push_back(*p++);
        if (tok.empty()) return fail("unexpected character");
        char* e = nullptr;
        v.kind = Json::NUM;
        v.num = strtod(tok.c_str(), &e);
        if (!e || *e) return fail("bad number");
        return true;
    }
};

bool parse_json(const std::string& text, Json& out, std::string& err) {
    JsonParser ps{text.data(), text.data() + text.size(), {}};
    if (!ps.value(out, 0)) {
        err = ps.err;
        return false;
    }
    ps.ws();
    if (ps.p != ps.end) {
        err = "trailing characters";
        return false;
    }
    return true;
}

bool read_text(const std::string& path, std::string& out) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return false;
    char buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
    fclose(f);
    return true;
}

/* ---- config.json -> bm_arch_t (reference config.c:128-297) ---- */

bool cfg_int(const Json* sec, const char* key, int* out) {
    const Json* v = sec->get(key);
    if (!v || v->kind != Json::NUM) return false;
    *out = (int)v->num;
    return true;
}

int arch_from_config(const char* dir, bm_arch_t* arch) {
    std::string text, err;
    const std::string path = std::string(dir) + "/config.json";
    if (!read_text(path, text)) {
        BMK_ERR("cannot read %s", path.c_str());
        return -1;
    }
    Json root;
    if (!parse_json(text, root, err) || root.kind != Json::OBJ) {
        BMK_ERR("%s: %s", path.c_str(), err.empty() ? "top-level value must be an object" : err.c_str());
        return -1;
    }
    const Json* sec = root.get("text_config");
    if (!sec || sec->kind != Json::OBJ) sec = &root;

    std::string model_type, architecture, act;
    const Json* mt = root.get("model_type");
    if (!mt || mt->kind != Json::STR) mt = sec->get("model_type");
    if (mt && mt->kind == Json::STR) model_type = mt->str;
    std::transform(model_type.begin(), model_type.end(), model_type.begin(), ::tolower);
    const Json* archs = root.get("architectures");
    if (!archs || archs->kind != Json::ARR) archs = sec->get("architectures");
    if (archs && archs->kind == Json::ARR && !archs->arr.empty() && archs->arr[0].kind == Json::STR)
        architecture = archs->arr[0].str;
    const bool llama = model_type == "llama" || model_type == "mistral" ||
                       (model_type.empty() && (architecture.find("Llama") != std::string::npos ||
                                               architecture.find("Mistral") != std::string::npos));
    if (!llama) {
        BMK_ERR("%s: model_type '%s' (%s): the MI355X path implements the llama family", path.c_str(),
                model_type.c_str(), architecture.c_str());
        return -1;
    }

    int hidden = 0, inter = 0, layers = 0, heads = 0, kv_heads = 0, vocab = 0, max_pos = 0, head_dim = 0;
    cfg_int(sec, "hidden_size", &hidden);
    cfg_int(sec, "intermediate_size", &inter);
    cfg_int(sec, "num_hidden_layers", &layers);
    cfg_int(sec, "num_attention_heads", &heads);
    cfg_int(sec, "num_key_value_heads", &kv_heads);
    cfg_int(sec, "vocab_size", &vocab);
    cfg_int(sec, "max_position_embeddings", &max_pos);
    cfg_int(sec, "head_dim", &head_dim);
    if (!hidden) cfg_int(sec, "n_embd", &hidden);
    if (!layers) cfg_int(sec, "n_layer", &layers);
    if (!heads) cfg_int(sec, "n_head", &heads);
    if (!max_pos) cfg_int(sec, "n_positions", &max_pos);
    if (!inter) cfg_int(sec, "n_inner", &inter);
    if (hidden <= 0 || inter <= 0 || layers <= 0 || heads <= 0 || vocab <= 0) {
        BMK_ERR("%s: missing dims hidden=%d ffn=%d layers=%d heads=%d vocab=%d", path.c_str(), hidden, inter, layers,
                heads, vocab);
        return -1;
    }
    auto flag = [&](const char* k) {
        const Json* v = sec->get(k);
        return v && v->kind == Json::BOOL && v->b;
    };
    const Json* an = sec->get("hidden_act");
    if (!an || an->kind != Json::STR) an = sec->get("hidden_activation");
    if (!an || an->kind != Json::STR) an = sec->get("activation_function");
    if (an && an->kind == Json::STR) act = an->str;

    memset(arch, 0, sizeof *arch);
    arch->dim = hidden;
    arch->hidden_dim = inter;
    arch->n_layers = layers;
    arch->n_heads = heads;
    arch->n_kv_heads = kv_heads > 0 ? kv_heads : heads;
    arch->vocab_size = arch->padded_vocab_size = vocab;
    arch->max_seq_len = max_pos > 0 ? max_pos : 2048;
    arch->head_dim = head_dim;
    arch->norm = sec->get("rms_norm_eps") ? BM_NORM_RMSNORM : BM_NORM_LAYERNORM;
    arch->activation =
        (act.find("silu") != std::string::npos || act.find("swiglu") != std::string::npos) ? BM_ACT_SWIGLU : BM_ACT_GELU;
    const Json* theta = sec->get("rope_theta");
    arch->pos_enc = theta && theta->kind == Json::NUM ? BM_POS_ROPE : BM_POS_LEARNED;
    arch->attention = arch->n_kv_heads < arch->n_heads ? BM_ATTN_GQA : BM_ATTN_MHA;
    arch->bias = flag("attention_bias") || flag("mlp_bias");
    arch->weight_tie = flag("tie_word_embeddings");
    arch->gated_mlp = arch->activation == BM_ACT_SWIGLU;
    arch->rope_theta = theta && theta->kind == Json::NUM ? (float)theta->num : 10000.0f;
    float factor = 0.f, lo = 0.f, hi = 0.f, orig = 0.f;
    const Json* sc = sec->get("rope_scaling");
    if (sc && sc->kind == Json::OBJ) {
        const Json* rt = sc->get("rope_type");
        if (!rt || rt->kind != Json::STR) rt = sc->get("type");
        arch->rope_scaling = rt && rt->kind == Json::STR && rt->str == "llama3" ? BM_ROPE_LLAMA3 : BM_ROPE_NONE;
        auto num = [&](const char* k, float* o) {
            const Json* v = sc->get(k);
            if (v && v->kind == Json::NUM) *o = (float)v->num;
        };
        num("factor", &factor);
        num("low_freq_factor", &lo);
        num("high_freq_factor", &hi);
        num("original_max_position_embeddings", &orig);
        if (!(rt && rt->kind == Json::STR && rt->str == "llama3")) {
            BMK_ERR("%s: rope_scaling type other than llama3 is not implemented", path.c_str());
            return -1;
        }
    }
    arch->rope_factor = factor > 0.f ? factor : 1.0f;
    arch->rope_low_freq_factor = lo > 0.f ? lo : 1.0f;
    arch->rope_high_freq_factor = hi > 0.f ? hi : 4.0f;
    arch->rope_original_max = orig > 0.f ? orig : (float)(max_pos > 0 ? max_pos : 8192);
    arch->precision = BM_PRECISION_FP32;
    return 0;
}

/* ---- safetensors ---- */

struct StTensor {
    int bf16;
    std::vector<long> shape;
    const unsigned char* data;
    size_t bytes;
};

struct StFile {
    void* base = MAP_FAILED;
    size_t size = 0;
    ~StFile() {
        if (base != MAP_FAILED) munmap(base, size);
    }
};

struct StSet {
    std::vector<std::unique_ptr<StFile>> files;
    std::map<std::string, StTensor> tensors;

    int add(const std::string& path) {
        const int fd = open(path.c_str(), O_RDONLY);
        if (fd < 0) {
            BMK_ERR("cannot open %s", path.c_str());
            return -1;
        }
        struct stat sb;
        if (fstat(fd, &sb) != 0 || sb.st_size < 8) {
            close(fd);
            BMK_ERR("%s: not a safetensors file", path.c_str());
            return -1;
        }
        std::unique_ptr<StFile> f(new StFile);
        f->size = (size_t)sb.st_size;
        f->base = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
        close(fd);
        if (f->base == MAP_FAILED) {
            BMK_ERR("mmap %s failed", path.c_str());
            return -1;
        }
        const unsigned char* b = (const unsigned char*)f->base;
        unsigned long long hlen = 0;
        for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | b[i]; /* little-endian u64 */
        if (hlen > f->size - 8) {
            BMK_ERR("%s: header length %llu beyond the file", path.c_str(), hlen);
            return -1;
        }
        Json h;
        std::string err;
        if (!parse_json(std::string((const char*)b + 8, (size_t)hlen), h, err) || h.kind != Json::OBJ) {
            BMK_ERR("%s: bad header: %s", path.c_str(), err.c_str());
            return -1;
        }
        const unsigned char* data = b + 8 + hlen;
        const size_t data_size = f->size - 8 - (size_t)hlen;
        for (const auto& kv : h.obj) {
            if (kv.first == "__metadata__") continue;
            const Json* dt = kv.second.get("dtype");
            const Json* sh = kv.second.get("shape");
            const Json* off = kv.second.get("data_offsets");
            if (!dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !off || off->kind != Json::ARR ||
                off->arr.size() != 2) {
                BMK_ERR("%s: bad entry %s", path.c_str(), kv.first.c_str());
                return -1;
            }
            StTensor t;
            if (dt->str == "BF16") t.bf16 = 1;
            else if (dt->str == "F32") t.bf16 = 0;
            else continue; /* other dtypes are not weights this path reads */
            const double o0 = off->arr[0].num, o1 = off->arr[1].num;
            if (o0 < 0 || o1 < o0 || o1 > (double)data_size) {
                BMK_ERR("%s: tensor %s outside the data section", path.c_str(), kv.first.c_str());
                return -1;
            }
            size_t n = 1;
            for (const Json& d : sh->arr) {
                t.shape.push_back((long)d.num);
                n *= (size_t)d.num;
            }
            t.data = data + (size_t)o0;
            t.bytes = (size_t)(o1 - o0);
            if (t.bytes != n * (t.bf16 ? 2 : 4)) {
                BMK_ERR("%s: tensor %s holds %zu bytes for %zu elements", path.c_str(), kv.first.c_str(), t.bytes, n);
                return -1;
            }
            tensors[kv.first] = t;
        }
        files.push_back(std::move(f));
        return 0;
    }

    int open_dir(const char* dir) {
        std::string text;
        const std::string idx = std::string(dir) + "/model.safetensors.index.json";
        if (read_text(idx, text)) {
            Json root;
            std::string err;
            if (!parse_json(text, root, err)) {
                BMK_ERR("%s: %s", idx.c_str(), err.c_str());
                return -1;
            }
            const Json* map = root.get("weight_map");
            if (!map || map->kind != Json::OBJ) {
                BMK_ERR("%s: missing weight_map", idx.c_str());
                return -1;
            }
            std::vector<std::string> shards;
            for (const auto& kv : map->obj)
                if (kv.second.kind == Json::STR &&
                    std::find(shards.begin(), shards.end(), kv.second.str) == shards.end())
                    shards.push_back(kv.second.str);
            if (shards.empty()) {
                BMK_ERR("%s: weight_map names no shard", idx.c_str());
                return -1;
            }
            for (const auto& sh : shards)
                if (add(std::string(dir) + "/" + sh)) return -1;
            return 0;
        }
        DIR* d = opendir(dir);
        if (!d) {
            BMK_ERR("cannot open directory %s", dir);
            return -1;
        }
        std::vector<std::string> names;
        while (struct dirent* de = readdir(d)) {
            const std::string n = de->d_name;
            if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) names.push_back(n);
        }
        closedir(d);
        std::sort(names.begin(), names.end());
        if (names.empty()) {
            BMK_ERR("%s: no .safetensors file", dir);
            return -1;
        }
        for (const auto& n : names)
            if (add(std::string(dir) + "/" + n)) return -1;
        return 0;
    }

    const StTensor* find(const std::string& name) const {
        auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }
};

} // namespace

extern "C" int bm_model_set_tensor_bf16(bm_model_t* model, const char* name, const uint16_t* data, size_t n);

/* One engine tensor gathered from its per-layer checkpoint tensors (layers
 * back to back, the reference's grouping by matrix type), fp32 or bf16. */
static int load_group(bm_model_t* m, const StSet& set, const char* engine_name, const std::vector<std::string>& names,
                      size_t per, bool keep_bf16) {
    bool any_bf16 = false;
    for (const auto& n : names) {
        const StTensor* t = set.find(n);
        if (!t) {
            BMK_ERR("checkpoint: tensor %s missing", n.c_str());
            return -1;
        }
        if (t->bytes != per * (t->bf16 ? 2 : 4)) {
            BMK_ERR("checkpoint: tensor %s holds %zu bytes, expected %zu elements", n.c_str(), t->bytes, per);
            return -1;
        }
        any_bf16 |= t->bf16 != 0;
    }
    const size_t total = per * names.size();
    if (keep_bf16 && any_bf16) {
        /* every part bf16 (an fp32 part is rounded to bf16 only if mixed, which
         * checkpoints do not do; reject it instead) */
        std::vector<uint16_t> buf(total);
        for (size_t i = 0; i < names.size(); i++) {
            const StTensor* t = set.find(names[i]);
            if (!t->bf16) {
                BMK_ERR("checkpoint: %s mixes F32 and BF16 tensors", engine_name);
                return -1;
            }
            memcpy(buf.data() + i * per, t->data, per * 2);
        }
        return bm_model_set_tensor_bf16(m, engine_name, buf.data(), total);
    }
    std::vector<float> buf(total);
    for (size_t i = 0; i < names.size(); i++) {
        const StTensor* t = set.find(names[i]);
        float* dst = buf.data() + i * per;
        if (t->bf16) {
            const uint16_t* s = (const uint16_t*)t->data;
            for (size_t j = 0; j < per; j++) {
                const uint32_t u = (uint32_t)s[j] << 16;
                memcpy(dst + j, &u, 4);
            }
        } else {
            memcpy(dst, t->data, per * 4);
        }
    }
    return bm_model_set_tensor(m, engine_name, buf.data(), total);
}

static int load_tensors(bm_model_t* m, const bm_arch_t* a, const StSet& set) {
    const int L = a->n_layers, D = a->dim, H = a->hidden_dim, NH = a->n_heads, NKV = a->n_kv_heads;
    const int HD = a->head_dim > 0 ? a->head_dim : D / NH;
    const size_t V = (size_t)a->vocab_size;
    auto layer_names = [&](const char* suffix) {
        std::vector<std::string> v;
        for (int l = 0; l < L; l++) v.push_back("model.layers." + std::to_string(l) + "." + suffix);
        return v;
    };
    struct G {
        const char* engine;
        const char* suffix;
        size_t per;
        bool q8;
    } groups[] = {
        {"ln1", "input_layernorm.weight", (size_t)D, false},
        {"wq", "self_attn.q_proj.weight", (size_t)NH * HD * D, true},
        {"wk", "self_attn.k_proj.weight", (size_t)NKV * HD * D, true},
        {"wv", "self_attn.v_proj.weight", (size_t)NKV * HD * D, true},
        {"wo", "self_attn.o_proj.weight", (size_t)D * NH * HD, true},
        {"ln2", "post_attention_layernorm.weight", (size_t)D, false},
        {"w_gate", "mlp.gate_proj.weight", (size_t)H * D, true},
        {"w_up", "mlp.up_proj.weight", (size_t)H * D, true},
        {"w_down", "mlp.down_proj.weight", (size_t)D * H, true},
    };
    if (load_group(m, set, "token_embedding", {"model.embed_tokens.weight"}, V * D, false)) return -1;
    for (const G& g : groups)
        if (load_group(m, set, g.engine, layer_names(g.suffix), g.per, g.q8)) return -1;
    if (load_group(m, set, "lnf", {"model.norm.weight"}, (size_t)D, false)) return -1;
    if (!a->weight_tie && load_group(m, set, "lm_head", {"lm_head.weight"}, V * D, false)) return -1;
    return 0;
}

/* The arch a checkpoint directory describes: config.json, with weight_tie
 * set when the tensors hold no lm_head (reference checkpoint_st.c:450-462). */
static int checkpoint_arch(const char* dir, StSet& set, bm_arch_t* arch) {
    if (arch_from_config(dir, arch)) return -1;
    if (set.open_dir(dir)) return -1;
    if (!set.find("lm_head.weight")) arch->weight_tie = 1;
    return 0;
}

extern "C" int bm_arch_from_checkpoint(const char* dir, bm_arch_t* arch) {
    if (!dir || !arch) return -1;
    StSet set;
    return checkpoint_arch(dir, set, arch);
}

extern "C" bm_model_t* bm_load_model(bm_context_t* ctx, const char* dir) {
    if (!ctx || !dir) return nullptr;
    StSet set;
    bm_arch_t arch;
    if (checkpoint_arch(dir, set, &arch)) return nullptr;
    bm_model_t* m = bm_create_model(ctx, &arch);
    if (!m) return nullptr;
    if (load_tensors(m, &arch, set)) {
        bm_destroy_model(m);
        return nullptr;
    }
    return m;
}

/* Reference include/baremetal.h:127 / api.c:45-49: weights of a model from a
 * checkpoint directory.  The model's shape must be the one the directory's
 * config.json describes. */
extern "C" int bm_model_arch(const bm_model_t* m, bm_arch_t* out);
extern "C" void bm_load_weights(bm_model_t* m, const char* dir) {
    if (!m || !dir) return;
    StSet set;
    bm_arch_t want, have;
    if (checkpoint_arch(dir, set, &want) || bm_model_arch(m, &have)) {
        BMK_ERR("bm_load_weights: failed to load weights from %s", dir);
        return;
    }
    const int hd_w = want.head_dim > 0 ? want.head_dim : want.dim / want.n_heads;
    const int hd_h = have.head_dim > 0 ? have.head_dim : have.dim / have.n_heads;
    if (want.dim != have.dim || want.hidden_dim != have.hidden_dim || want.n_layers != have.n_layers ||
        want.n_heads != have.n_heads || want.n_kv_heads != have.n_kv_heads || want.vocab_size != have.vocab_size ||
        hd_w != hd_h || (want.weight_tie != 0) != (have.weight_tie != 0)) {
        BMK_ERR("bm_load_weights: %s describes another shape than the model's", dir);
        return;
    }
    if (load_tensors(m, &want, set)) BMK_ERR("bm_load_weights: failed to load weights from %s", dir);
}
