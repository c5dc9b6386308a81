// st_loader.cpp — the model's weights on disk: safetensors files memory-mapped and looked up by tensor name, loaded
// into the GPU tier (moe_gpu) and the decode model (moe_model), and the engine's expert placement file.
//
// Replaces the engine's Weights (track2_opt/solar_engine/src/host.rs:78-117: every *.safetensors file of the model
// directory, in name order, memory-mapped; tensors by their HF names, bf16 zero-copy) and its placement.json reader
// (main.rs:455; format moe_offload/placement.py:3: [layer][tier] -> expert ids in slot order).
//
// safetensors format: an 8-byte little-endian header length N, then N bytes of JSON
//   {"<name>": {"dtype": "BF16", "shape": [d0, d1, ...], "data_offsets": [begin, end]}, ..., "__metadata__": {...}}
// then the data block, offsets relative to its start.  The JSON parser below reads exactly that subset (objects,
// arrays, strings, integers; other values are skipped) and rejects anything malformed.
#include <dirent.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <stdint.h>

#include <algorithm>
#include <initializer_list>
#include <string>
#include <unordered_map>
#include <vector>

#include "moe_gpu.h"

namespace {

struct Tensor {
    const unsigned char* data = nullptr;
    size_t nbytes = 0;
    int dtype = -1;
    std::vector<int64_t> shape;
};

struct Mapping {
    void* base = nullptr;
    size_t len = 0;
};

thread_local std::string t_err = "no error";

int sfail(std::string* err, int code, const char* fmt, ...) {
    char buf[768];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    (err ? *err : t_err) = buf;
    return code;
}

int dtype_code(const std::string& s) {
    if (s == "BF16") return MOE_ST_BF16;
    if (s == "F32") return MOE_ST_F32;
    if (s == "F16") return MOE_ST_F16;
    if (s == "I8") return MOE_ST_I8;
    if (s == "I32") return MOE_ST_I32;
    if (s == "I64") return MOE_ST_I64;
    if (s == "U8") return MOE_ST_U8;
    return -1;
}
size_t dtype_size(int d) {
    switch (d) {
        case MOE_ST_BF16: case MOE_ST_F16: return 2;
        case MOE_ST_F32: case MOE_ST_I32: return 4;
        case MOE_ST_I64: return 8;
        case MOE_ST_I8: case MOE_ST_U8: return 1;
        default: return 0;
    }
}

// Minimal JSON reader over [p, e).
struct Json {
    const char* p;
    const char* e;
    bool ok = true;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    bool eat(char c) {
        ws();
        if (p < e && *p == c) {
            p++;
            return true;
        }
        return false;
    }
    bool str(std::string* out) {
        ws();
        if (p >= e || *p != '"') return ok = false;
        p++;
        std::string s;
        while (p < e && *p != '"') {
            if (*p == '\\') {  // escapes: kept verbatim except \" and \\ (tensor names use neither)
                if (p + 1 >= e) return ok = false;
                p++;
            }
            s.push_back(*p++);
        }
        if (p >= e) return ok = false;
        p++;
        if (out) *out = std::move(s);
        return true;
    }
    bool integer(int64_t* out) {
        ws();
        const char* q = p;
        bool neg = false;
        if (q < e && *q == '-') {
            neg = true;
            q++;
        }
        if (q >= e || *q < '0' || *q > '9') return ok = false;
        int64_t v = 0;
        while (q < e && *q >= '0' && *q <= '9') {
            if (v > (INT64_MAX - 9) / 10) return ok = false;
            v = v * 10 + (*q++ - '0');
        }
        p = q;
        *out = neg ? -v : v;
        return true;
    }
    bool int_array(std::vector<int64_t>* out) {
        if (!eat('[')) return ok = false;
        out->clear();
        if (eat(']')) return true;
        do {
            int64_t v;
            if (!integer(&v)) return false;
            out->push_back(v);
        } while (eat(','));
        return eat(']') || (ok = false);
    }
    bool skip_value(int depth = 0) {  // any JSON value
        ws();
        if (p >= e || depth > 32) return ok = false;
        if (*p == '"') return str(nullptr);
        if (*p == '{' || *p == '[') {
            const char close = *p == '{' ? '}' : ']';
            const bool obj = *p == '{';
            p++;
            if (eat(close)) return true;
            do {
                if (obj) {
                    if (!str(nullptr) || !eat(':')) return ok = false;
                }
                if (!skip_value(depth + 1)) return false;
            } while (eat(','));
            return eat(close) || (ok = false);
        }
        while (p < e && *p != ',' && *p != '}' && *p != ']') p++;  // number, true, false, null
        return true;
    }
};

}  // namespace

struct moe_st {
    std::vector<Mapping> maps;
    std::unordered_map<std::string, Tensor> tensors;
    std::string err = "no error";
};

namespace {

// One file: map it, parse its header, add its tensors (a name seen in an earlier file is replaced, as the engine's
// HashMap insert does).
int add_file(moe_st* st, const std::string& path) {
    const int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) return sfail(&st->err, MOE_GPU_EINVAL, "cannot open %s", path.c_str());
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 8) {
        close(fd);
        return sfail(&st->err, MOE_GPU_EINVAL, "%s: too short for a safetensors file", path.c_str());
    }
    const size_t len = (size_t)sb.st_size;
    void* base = mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (base == MAP_FAILED) return sfail(&st->err, MOE_GPU_EINVAL, "%s: mmap failed", path.c_str());
    st->maps.push_back({base, len});
    const unsigned char* b = static_cast<const unsigned char*>(base);
    uint64_t n = 0;
    for (int i = 7; i >= 0; i--) n = (n << 8) | b[i];
    if (n > len - 8) return sfail(&st->err, MOE_GPU_EINVAL, "%s: header length %llu beyond the file", path.c_str(),
                                  (unsigned long long)n);
    const unsigned char* data0 = b + 8 + n;
    const size_t data_len = len - 8 - n;
    Json j{reinterpret_cast<const char*>(b + 8), reinterpret_cast<const char*>(b + 8 + n)};
    if (!j.eat('{')) return sfail(&st->err, MOE_GPU_EINVAL, "%s: header is not a JSON object", path.c_str());
    if (!j.eat('}')) {
        do {
            std::string name;
            if (!j.str(&name) || !j.eat(':')) return sfail(&st->err, MOE_GPU_EINVAL, "%s: bad header", path.c_str());
            if (name == "__metadata__") {
                if (!j.skip_value()) return sfail(&st->err, MOE_GPU_EINVAL, "%s: bad __metadata__", path.c_str());
                continue;
            }
            if (!j.eat('{')) return sfail(&st->err, MOE_GPU_EINVAL, "%s: tensor %s is not an object", path.c_str(),
                                          name.c_str());
            Tensor t;
            std::string dt;
            std::vector<int64_t> off;
            bool have_dt = false, have_shape = false, have_off = false;
            if (!j.eat('}')) {
                do {
                    std::string key;
                    if (!j.str(&key) || !j.eat(':')) return sfail(&st->err, MOE_GPU_EINVAL, "%s: bad entry %s",
                                                                  path.c_str(), name.c_str());
                    if (key == "dtype") have_dt = j.str(&dt);
                    else if (key == "shape") have_shape = j.int_array(&t.shape);
                    else if (key == "data_offsets") have_off = j.int_array(&off);
                    else if (!j.skip_value()) break;
                    if (!j.ok) break;
                } while (j.eat(','));
                if (!j.ok || !j.eat('}'))
                    return sfail(&st->err, MOE_GPU_EINVAL, "%s: bad entry %s", path.c_str(), name.c_str());
            }
            if (!have_dt || !have_shape || !have_off || off.size() != 2)
                return sfail(&st->err, MOE_GPU_EINVAL, "%s: %s lacks dtype, shape or data_offsets", path.c_str(),
                             name.c_str());
            t.dtype = dtype_code(dt);
            if (t.dtype < 0)
                return sfail(&st->err, MOE_GPU_EINVAL, "%s: %s has unsupported dtype %s", path.c_str(), name.c_str(),
                             dt.c_str());
            size_t count = 1;
            for (int64_t d : t.shape) {
                if (d < 0) return sfail(&st->err, MOE_GPU_EINVAL, "%s: %s has a negative dim", path.c_str(), name.c_str());
                count *= (size_t)d;
            }
            if (off[0] < 0 || off[1] < off[0] || (size_t)off[1] > data_len ||
                (size_t)(off[1] - off[0]) != count * dtype_size(t.dtype))
                return sfail(&st->err, MOE_GPU_EINVAL, "%s: %s data_offsets [%lld, %lld] do not match its shape or the "
                             "file", path.c_str(), name.c_str(), (long long)off[0], (long long)off[1]);
            t.data = data0 + off[0];
            t.nbytes = (size_t)(off[1] - off[0]);
            st->tensors[name] = std::move(t);
        } while (j.eat(','));
        if (!j.eat('}')) return sfail(&st->err, MOE_GPU_EINVAL, "%s: header object not closed", path.c_str());
    }
    return MOE_GPU_OK;
}

// A bf16 tensor of exactly the given shape.
int want_bf16(moe_st* st, const std::string& name, std::initializer_list<int64_t> shape, const uint16_t** out) {
    auto it = st->tensors.find(name);
    if (it == st->tensors.end()) return sfail(&st->err, MOE_GPU_EINVAL, "missing tensor %s", name.c_str());
    const Tensor& t = it->second;
    if (t.dtype != MOE_ST_BF16) return sfail(&st->err, MOE_GPU_EINVAL, "%s is not bf16", name.c_str());
    if (!std::equal(t.shape.begin(), t.shape.end(), shape.begin(), shape.end())) {
        std::string got, exp;
        for (int64_t d : t.shape) got += std::to_string(d) + " ";
        for (int64_t d : shape) exp += std::to_string(d) + " ";
        return sfail(&st->err, MOE_GPU_EINVAL, "%s has shape [ %s] instead of [ %s]", name.c_str(), got.c_str(),
                     exp.c_str());
    }
    *out = reinterpret_cast<const uint16_t*>(t.data);
    return MOE_GPU_OK;
}

std::string lname(int l, const char* n) { return "model.layers." + std::to_string(l) + "." + n; }

}  // namespace

extern "C" {

int moe_st_open(const char* dir, moe_st** out) {
    if (!out) return sfail(nullptr, MOE_GPU_EINVAL, "NULL out");
    *out = nullptr;
    if (!dir) return sfail(nullptr, MOE_GPU_EINVAL, "NULL directory");
    DIR* d = opendir(dir);
    if (!d) return sfail(nullptr, MOE_GPU_EINVAL, "cannot open directory %s", dir);
    std::vector<std::string> files;
    while (struct dirent* de = readdir(d)) {
        const std::string n = de->d_name;
        if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) files.push_back(n);
    }
    closedir(d);
    std::sort(files.begin(), files.end());  // the engine's files.sort() (host.rs:86)
    if (files.empty()) return sfail(nullptr, MOE_GPU_EINVAL, "no *.safetensors file in %s", dir);
    moe_st* st = new moe_st();
    for (const std::string& f : files) {
        const int rc = add_file(st, std::string(dir) + "/" + f);
        if (rc != MOE_GPU_OK) {
            t_err = st->err;
            moe_st_close(st);
            return rc;
        }
    }
    *out = st;
    return MOE_GPU_OK;
}

void moe_st_close(moe_st* st) {
    if (!st) return;
    for (const Mapping& m : st->maps) munmap(m.base, m.len);
    delete st;
}

const char* moe_st_last_error(const moe_st* st) { return st ? st->err.c_str() : t_err.c_str(); }

int moe_st_count(const moe_st* st) { return st ? (int)st->tensors.size() : 0; }

int moe_st_tensor(const moe_st* cst, const char* name, const void** data, size_t* nbytes, int* dtype, int64_t* shape,
                  int* ndim) {
    moe_st* st = const_cast<moe_st*>(cst);
    if (!st || !name) return sfail(nullptr, MOE_GPU_EINVAL, "NULL argument");
    auto it = st->tensors.find(name);
    if (it == st->tensors.end()) return sfail(&st->err, MOE_GPU_EINVAL, "missing tensor %s", name);
    const Tensor& t = it->second;
    if (data) *data = t.data;
    if (nbytes) *nbytes = t.nbytes;
    if (dtype) *dtype = t.dtype;
    if (ndim) {
        const int cap = *ndim;
        *ndim = (int)t.shape.size();
        if (shape)
            for (int i = 0; i < std::min(cap, *ndim); i++) shape[i] = t.shape[i];
    }
    return MOE_GPU_OK;
}

int moe_st_load_moe_layer(const moe_st* cst, moe_gpu* ctx, int model_layer, int tier_layer, const int32_t* experts,
                          int n_experts) {
    moe_st* st = const_cast<moe_st*>(cst);
    if (!st || !ctx) return sfail(nullptr, MOE_GPU_EINVAL, "NULL argument");
    int H = 0, F = 0, E = 0, k = 0, S = 0, L = 0;
    int rc = moe_gpu_get_shape(ctx, &H, &F, &E, &k, &S, &L);
    if (rc) return sfail(&st->err, rc, "moe_gpu_get_shape: %s", moe_gpu_last_error(ctx));
    if (tier_layer < 0 || tier_layer >= L) return sfail(&st->err, MOE_GPU_EINVAL, "tier layer %d outside [0, %d)",
                                                        tier_layer, L);
    const int l = model_layer;
    // router and its selection bias (main.rs:519; a model without the bias routes on the logits alone)
    const uint16_t* wr;
    if ((rc = want_bf16(st, lname(l, "mlp.gate.weight"), {E, H}, &wr))) return rc;
    std::vector<float> bias;
    auto bi = st->tensors.find(lname(l, "mlp.gate.e_score_correction_bias"));
    if (bi != st->tensors.end()) {
        const Tensor& t = bi->second;
        if (t.shape.size() != 1 || t.shape[0] != E || (t.dtype != MOE_ST_F32 && t.dtype != MOE_ST_BF16))
            return sfail(&st->err, MOE_GPU_EINVAL, "%s: want [%d] fp32 or bf16", bi->first.c_str(), E);
        bias.resize(E);
        for (int e = 0; e < E; e++) {
            if (t.dtype == MOE_ST_F32) memcpy(&bias[e], t.data + 4 * e, 4);
            else {
                const uint32_t v = (uint32_t)(t.data[2 * e] | (t.data[2 * e + 1] << 8)) << 16;
                memcpy(&bias[e], &v, 4);
            }
        }
    }
    if ((rc = moe_gpu_load_router(ctx, tier_layer, wr, bias.empty() ? nullptr : bias.data())))
        return sfail(&st->err, rc, "moe_gpu_load_router: %s", moe_gpu_last_error(ctx));
    // shared experts: one (mlp.shared_experts.*) or several (mlp.shared_experts.{s}.*); the engine's Solar has one
    for (int s = 0; s < S; s++) {
        const std::string p = S == 1 ? lname(l, "mlp.shared_experts.") : lname(l, "mlp.shared_experts.") +
                                                                            std::to_string(s) + ".";
        const uint16_t *g, *u, *d;
        if ((rc = want_bf16(st, p + "gate_proj.weight", {F, H}, &g)) ||
            (rc = want_bf16(st, p + "up_proj.weight", {F, H}, &u)) ||
            (rc = want_bf16(st, p + "down_proj.weight", {H, F}, &d)))
            return rc;
        if ((rc = moe_gpu_load_shared(ctx, tier_layer, s, g, u, d)))
            return sfail(&st->err, rc, "moe_gpu_load_shared: %s", moe_gpu_last_error(ctx));
    }
    // routed experts (host.rs:111-116): the listed ones, or every one
    const int n = n_experts < 0 ? E : n_experts;
    for (int i = 0; i < n; i++) {
        const int e = n_experts < 0 ? i : experts[i];
        if (e < 0 || e >= E) return sfail(&st->err, MOE_GPU_EINVAL, "expert id %d outside [0, %d)", e, E);
        const std::string p = lname(l, "mlp.experts.") + std::to_string(e) + ".";
        const uint16_t *g, *u, *d;
        if ((rc = want_bf16(st, p + "gate_proj.weight", {F, H}, &g)) ||
            (rc = want_bf16(st, p + "up_proj.weight", {F, H}, &u)) ||
            (rc = want_bf16(st, p + "down_proj.weight", {H, F}, &d)))
            return rc;
        if ((rc = moe_gpu_load_expert(ctx, tier_layer, e, g, u, d)))
            return sfail(&st->err, rc, "moe_gpu_load_expert: %s", moe_gpu_last_error(ctx));
    }
    return MOE_GPU_OK;
}

int moe_st_load_model(const moe_st* cst, moe_model* m) {
    moe_st* st = const_cast<moe_st*>(cst);
    if (!st || !m) return sfail(nullptr, MOE_GPU_EINVAL, "NULL argument");
    moe_model_config c;
    int rc = moe_model_get_config(m, &c);
    if (rc) return sfail(&st->err, rc, "moe_model_get_config: %s", moe_model_last_error(m));
    const int64_t H = c.H, QD = (int64_t)c.n_q_heads * c.head_dim, KVD = (int64_t)c.n_kv_heads * c.head_dim;
    for (int l = 0; l < c.n_layers; l++) {  // the dense weights of main.rs:466-468
        const uint16_t *w_in, *wq, *wk, *wv, *wo, *w_post;
        if ((rc = want_bf16(st, lname(l, "input_layernorm.weight"), {H}, &w_in)) ||
            (rc = want_bf16(st, lname(l, "self_attn.q_proj.weight"), {QD, H}, &wq)) ||
            (rc = want_bf16(st, lname(l, "self_attn.k_proj.weight"), {KVD, H}, &wk)) ||
            (rc = want_bf16(st, lname(l, "self_attn.v_proj.weight"), {KVD, H}, &wv)) ||
            (rc = want_bf16(st, lname(l, "self_attn.o_proj.weight"), {H, QD}, &wo)) ||
            (rc = want_bf16(st, lname(l, "post_attention_layernorm.weight"), {H}, &w_post)))
            return rc;
        if ((rc = moe_model_load_layer(m, l, w_in, wq, wk, wv, wo, w_post)))
            return sfail(&st->err, rc, "moe_model_load_layer: %s", moe_model_last_error(m));
        if ((rc = moe_st_load_moe_layer(st, moe_model_experts(m), l, l, nullptr, -1))) return rc;
    }
    const uint16_t *emb, *lm, *w_final;
    if ((rc = want_bf16(st, "model.embed_tokens.weight", {c.vocab, H}, &emb)) ||
        (rc = want_bf16(st, "lm_head.weight", {c.vocab, H}, &lm)) ||
        (rc = want_bf16(st, "model.norm.weight", {H}, &w_final)))
        return rc;
    if ((rc = moe_model_load_embedding(m, emb))) return sfail(&st->err, rc, "load_embedding: %s", moe_model_last_error(m));
    if ((rc = moe_head_load(moe_model_head(m), lm, w_final)))
        return sfail(&st->err, rc, "moe_head_load failed");
    return MOE_GPU_OK;
}

// placement.json: a JSON array over layers of arrays over tiers of arrays of expert ids.
int moe_placement_read(const char* path, int layer, int tier, int32_t* ids, int cap, int* n) {
    if (!path || !n) return sfail(nullptr, MOE_GPU_EINVAL, "NULL argument");
    FILE* f = fopen(path, "rb");
    if (!f) return sfail(nullptr, MOE_GPU_EINVAL, "cannot open %s", path);
    std::string text;
    char buf[65536];
    size_t r;
    while ((r = fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, r);
    fclose(f);
    Json j{text.data(), text.data() + text.size()};
    if (!j.eat('[')) return sfail(nullptr, MOE_GPU_EINVAL, "%s: not a JSON array", path);
    int li = 0;
    bool found = false;
    if (!j.eat(']')) {
        do {
            if (li != layer) {
                if (!j.skip_value()) return sfail(nullptr, MOE_GPU_EINVAL, "%s: bad layer %d", path, li);
            } else {
                if (!j.eat('[')) return sfail(nullptr, MOE_GPU_EINVAL, "%s: layer %d is not an array", path, li);
                int ti = 0;
                if (!j.eat(']')) {
                    do {
                        if (ti != tier) {
                            if (!j.skip_value()) return sfail(nullptr, MOE_GPU_EINVAL, "%s: bad tier", path);
                        } else {
                            std::vector<int64_t> v;
                            if (!j.int_array(&v)) return sfail(nullptr, MOE_GPU_EINVAL, "%s: bad id list", path);
                            *n = (int)v.size();
                            if (ids) {
                                if ((int)v.size() > cap)
                                    return sfail(nullptr, MOE_GPU_EINVAL, "%s: %d ids, room for %d", path, *n, cap);
                                for (size_t i = 0; i < v.size(); i++) ids[i] = (int32_t)v[i];
                            }
                            found = true;
                        }
                        ti++;
                    } while (j.eat(','));
                    if (!j.eat(']')) return sfail(nullptr, MOE_GPU_EINVAL, "%s: layer %d not closed", path, li);
                }
            }
            li++;
        } while (j.eat(','));
        if (!j.eat(']')) return sfail(nullptr, MOE_GPU_EINVAL, "%s: not closed", path);
    }
    if (!found) return sfail(nullptr, MOE_GPU_EINVAL, "%s: no tier %d of layer %d (%d layers)", path, tier, layer, li);
    return MOE_GPU_OK;
}

}  // extern "C"
