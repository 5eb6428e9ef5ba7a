// model.hip -- loading a decoder from a safetensors checkpoint with INT8 or
// FP8 E4M3 weights (host code).
//
// Reference: load_config src/inference/model.c:32-143 (HF config.json keys,
// "text_config" nesting, defaults, norm_eps forced to 1e-5), load_model /
// parse_header src/loader/loader_io.c:44-57, src/loader/loader_parse.c:28-110
// (safetensors: 8-byte header length, JSON header, data), the weight mapping
// by name substrings src/inference/model.c:180-265 (LLaMA and HF names, weight
// tying of the output to the embedding).
//
// The reference maps every tensor as BF16 whatever its dtype
// (loader_parse.c:48) and has no quantized tensor types (tensor.h:21-25).
// Here the dtype is honoured:
//   I8 / F8_E4M3   weight codes, with a per-output-row F32 scale tensor named
//                  "<weight name>_scale" (shape [rows] or [rows, 1]);
//   BF16 / F16 / F32  quantized per row on load with the library's codecs
//                  (quant_f32_to_int8 / quant_f32_to_fp8 semantics), to the
//                  kind of the options (INT8 or FP8);
// norm weights are kept as bf16 (F32 and F16 are rounded to bf16).  Every
// matrix of a model must end up one kind (the decoder streams one).
#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fcntl.h>
#include <string>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <vector>

#include "be42_common.h"

namespace be42 {

namespace {

// ---- config.json (load_config semantics) -----------------------------------

struct Conf {
    int dim = 0, hidden_dim = 0, n_layers = 0, n_heads = 0, n_kv_heads = 0, vocab = 0, head_dim = 0;
    float rope_theta = 0.0f, norm_eps = 0.0f;
};

void parse_int(const char *line, const char *key, int &dst)
{
    if (const char *k = strstr(line, key))
        if (const char *colon = strchr(k, ':'))
            dst = atoi(colon + 1);
}

void parse_float(const char *line, const char *key, float &dst)
{
    if (const char *k = strstr(line, key))
        if (const char *colon = strchr(k, ':'))
            dst = (float)strtod(colon + 1, nullptr);
}

// One pass over the lines: keys inside "text_config" (VLM files) or at the
// root; "vision_config" skipped; rope_theta inside "rope_parameters" too.
bool load_conf(const char *path, Conf &c, std::string &err)
{
    FILE *f = fopen(path, "r");
    if (!f) {
        err = std::string("cannot open config '") + path + "'";
        return false;
    }
    char line[1024];
    bool in_text = false, in_rope = false, in_vision = false;
    while (fgets(line, sizeof line, f)) {
        if (strstr(line, "\"text_config\": {")) {
            in_text = true;
            continue;
        }
        if (strstr(line, "\"vision_config\": {")) {
            in_vision = true;
            continue;
        }
        if (in_text && strstr(line, "\"rope_parameters\": {")) {
            in_rope = true;
            continue;
        }
        if (in_rope && strstr(line, "},")) {
            in_rope = false;
            continue;
        }
        if (in_vision && strstr(line, "},")) {
            in_vision = false;
            continue;
        }
        if (in_text && !in_rope && strstr(line, "},")) {
            in_text = false;
            continue;
        }
        if (in_vision)
            continue;
        if (in_rope) {
            parse_float(line, "\"rope_theta\":", c.rope_theta);
        } else {
            parse_int(line, "\"hidden_size\":", c.dim);
            parse_int(line, "\"intermediate_size\":", c.hidden_dim);
            parse_int(line, "\"num_hidden_layers\":", c.n_layers);
            parse_int(line, "\"num_attention_heads\":", c.n_heads);
            parse_int(line, "\"num_key_value_heads\":", c.n_kv_heads);
            parse_int(line, "\"vocab_size\":", c.vocab);
            parse_int(line, "\"head_dim\":", c.head_dim);
            if (!in_text) {
                parse_float(line, "\"rope_theta\":", c.rope_theta);
                parse_int(line, "\"dim\":", c.dim);
                parse_int(line, "\"n_layers\":", c.n_layers);
                parse_int(line, "\"n_heads\":", c.n_heads);
                parse_int(line, "\"n_kv_heads\":", c.n_kv_heads);
            }
        }
    }
    fclose(f);
    // the reference's defaults and overrides (model.c:112-140)
    if (c.dim == 0) c.dim = 3072;
    if (c.hidden_dim == 0) c.hidden_dim = 9216;
    if (c.n_layers == 0) c.n_layers = 26;
    if (c.n_heads == 0) c.n_heads = 32;
    if (c.n_kv_heads == 0) c.n_kv_heads = 8;
    if (c.vocab == 0) c.vocab = 131072;
    if (c.head_dim == 0)
        c.head_dim = c.dim > 0 && c.n_heads > 0 ? c.dim / c.n_heads : 128;
    if (c.rope_theta == 0.0f) c.rope_theta = 1000000.0f;
    c.norm_eps = 1e-5f;
    return true;
}

// ---- safetensors ------------------------------------------------------------

enum Dt { DT_BAD, DT_I8, DT_F8, DT_BF16, DT_F16, DT_F32 };

struct StTensor {
    std::string name;
    Dt dt = DT_BAD;
    std::vector<long long> shape;
    size_t begin = 0, end = 0;   // byte offsets in the data section
};

struct StFile {
    int fd = -1;
    void *map = nullptr;
    size_t size = 0;
    const uint8_t *data = nullptr;   // start of the data section
    size_t data_size = 0;
    std::vector<StTensor> tensors;
    ~StFile()
    {
        if (map && map != MAP_FAILED)
            munmap(map, size);
        if (fd >= 0)
            close(fd);
    }
    const StTensor *find(const std::string &n) const
    {
        for (const StTensor &t : tensors)
            if (t.name == n)
                return &t;
        return nullptr;
    }
};

Dt parse_dtype(const std::string &s)
{
    if (s == "I8") return DT_I8;
    if (s == "F8_E4M3") return DT_F8;
    if (s == "BF16") return DT_BF16;
    if (s == "F16") return DT_F16;
    if (s == "F32") return DT_F32;
    return DT_BAD;
}

size_t dt_size(Dt d) { return d == DT_F32 ? 4 : (d == DT_BF16 || d == DT_F16) ? 2 : 1; }

// A small reader of the header JSON: an object of objects with "dtype",
// "shape" and "data_offsets" (and "__metadata__", skipped).
struct Json {
    const char *p, *e;
    bool ok = true;
    void ws()
    {
        while (p < e && isspace((unsigned char)*p))
            p++;
    }
    bool lit(char c)
    {
        ws();
        if (p < e && *p == c) {
            p++;
            return true;
        }
        return false;
    }
    std::string str()
    {
        ws();
        std::string s;
        if (p >= e || *p != '"') {
            ok = false;
            return s;
        }
        p++;
        while (p < e && *p != '"') {
            if (*p == '\\' && p + 1 < e)
                p++;
            s += *p++;
        }
        if (p < e)
            p++;
        else
            ok = false;
        return s;
    }
    // an optionally signed decimal integer read within [p, e) (the header is
    // not NUL-terminated); values past 2^62 are an error
    long long num()
    {
        ws();
        bool neg = false;
        if (p < e && (*p == '-' || *p == '+'))
            neg = *p++ == '-';
        const char *d0 = p;
        long long v = 0;
        while (p < e && *p >= '0' && *p <= '9') {
            if (v > ((1LL << 62) - 9) / 10) {
                ok = false;
                return 0;
            }
            v = v * 10 + (*p++ - '0');
        }
        if (p == d0)
            ok = false;
        return neg ? -v : v;
    }
    void skip_value()
    {
        ws();
        if (p >= e) {
            ok = false;
            return;
        }
        if (*p == '"') {
            str();
        } else if (*p == '{' || *p == '[') {
            int depth = 0;
            bool in_s = false;
            for (; p < e; p++) {
                if (in_s) {
                    if (*p == '\\')
                        p++;
                    else if (*p == '"')
                        in_s = false;
                } else if (*p == '"') {
                    in_s = true;
                } else if (*p == '{' || *p == '[') {
                    depth++;
                } else if (*p == '}' || *p == ']') {
                    if (--depth == 0) {
                        p++;
                        return;
                    }
                }
            }
            ok = false;
        } else {
            while (p < e && *p != ',' && *p != '}' && *p != ']')
                p++;
        }
    }
};

bool open_st(const char *path, StFile &F, std::string &err)
{
    F.fd = open(path, O_RDONLY);
    if (F.fd < 0) {
        err = std::string("cannot open '") + path + "': " + strerror(errno);
        return false;
    }
    struct stat sb;
    if (fstat(F.fd, &sb) != 0 || sb.st_size < 8) {
        err = "not a safetensors file (too short)";
        return false;
    }
    F.size = (size_t)sb.st_size;
    F.map = mmap(nullptr, F.size, PROT_READ, MAP_PRIVATE, F.fd, 0);
    if (F.map == MAP_FAILED) {
        err = std::string("mmap failed: ") + strerror(errno);
        return false;
    }
    uint64_t hlen = 0;
    memcpy(&hlen, F.map, 8);
    if (hlen > F.size - 8) {
        err = "safetensors header length past the end of the file";
        return false;
    }
    const char *h = (const char *)F.map + 8;
    F.data = (const uint8_t *)F.map + 8 + hlen;
    F.data_size = F.size - 8 - hlen;
    Json J{h, h + hlen};
    if (!J.lit('{')) {
        err = "safetensors header is not a JSON object";
        return false;
    }
    if (J.lit('}'))
        return true;
    do {
        StTensor t;
        t.name = J.str();
        if (!J.ok || !J.lit(':'))
            break;
        if (t.name == "__metadata__") {
            J.skip_value();
            continue;
        }
        if (!J.lit('{')) {
            J.ok = false;
            break;
        }
        bool have_off = false;
        if (!J.lit('}')) {
            do {
                const std::string key = J.str();
                if (!J.ok || !J.lit(':'))
                    break;
                if (key == "dtype") {
                    t.dt = parse_dtype(J.str());
                } else if (key == "shape") {
                    if (!J.lit('[')) {
                        J.ok = false;
                        break;
                    }
                    if (!J.lit(']')) {
                        do
                            t.shape.push_back(J.num());
                        while (J.ok && J.lit(','));
                        if (!J.lit(']'))
                            J.ok = false;
                    }
                } else if (key == "data_offsets") {
                    if (!J.lit('[')) {
                        J.ok = false;
                        break;
                    }
                    t.begin = (size_t)J.num();
                    if (!J.lit(','))
                        J.ok = false;
                    t.end = (size_t)J.num();
                    if (!J.lit(']'))
                        J.ok = false;
                    have_off = true;
                } else {
                    J.skip_value();
                }
            } while (J.ok && J.lit(','));
            if (!J.lit('}'))
                J.ok = false;
        }
        if (!J.ok)
            break;
        size_t elems = 1, bytes = 0;
        bool wrap = false;
        for (long long d : t.shape)
            wrap |= __builtin_mul_overflow(elems, (size_t)(d > 0 ? d : 0), &elems);
        wrap |= t.dt != DT_BAD && __builtin_mul_overflow(elems, dt_size(t.dt), &bytes);
        if (!have_off || wrap || t.end < t.begin || t.end > F.data_size ||
            (t.dt != DT_BAD && t.end - t.begin != bytes)) {
            err = "tensor '" + t.name + "': data offsets do not match its shape and dtype";
            return false;
        }
        F.tensors.push_back(std::move(t));
    } while (J.lit(','));
    if (!J.ok) {
        err = "malformed safetensors header";
        return false;
    }
    return true;
}

// ---- the weight mapping (model.c:180-265) -----------------------------------

struct Mapped {
    // per layer: wq wk wv wo w1 w2 w3 attn_norm ffn_norm
    std::vector<const StTensor *> L[9];
    const StTensor *emb = nullptr, *norm = nullptr, *out = nullptr;
};

enum { M_WQ, M_WK, M_WV, M_WO, M_W1, M_W2, M_W3, M_AN, M_FN };

void map_names(const StFile &F, int n_layers, Mapped &M)
{
    for (auto &v : M.L)
        v.assign(n_layers, nullptr);
    for (const StTensor &t : F.tensors) {
        const char *name = t.name.c_str();
        if (strstr(name, "_scale"))
            continue;   // a scale tensor belongs to its weight
        if (const char *lm = strstr(name, "layers.")) {
            const int l = atoi(lm + 7);
            if (l < 0 || l >= n_layers)
                continue;
            int slot = -1;
            if (strstr(name, "attention.wq") || strstr(name, "self_attn.q_proj")) slot = M_WQ;
            else if (strstr(name, "attention.wk") || strstr(name, "self_attn.k_proj")) slot = M_WK;
            else if (strstr(name, "attention.wv") || strstr(name, "self_attn.v_proj")) slot = M_WV;
            else if (strstr(name, "attention.wo") || strstr(name, "self_attn.o_proj")) slot = M_WO;
            else if (strstr(name, "feed_forward.w1") || strstr(name, "mlp.gate_proj")) slot = M_W1;
            else if (strstr(name, "feed_forward.w2") || strstr(name, "mlp.down_proj")) slot = M_W2;
            else if (strstr(name, "feed_forward.w3") || strstr(name, "mlp.up_proj")) slot = M_W3;
            else if (strstr(name, "attention_norm") || strstr(name, "input_layernorm")) slot = M_AN;
            else if (strstr(name, "ffn_norm") || strstr(name, "post_attention_layernorm")) slot = M_FN;
            if (slot >= 0)
                M.L[slot][l] = &t;
        } else if (t.name == "tok_embeddings.weight" || t.name == "model.embed_tokens.weight") {
            M.emb = &t;
        } else if (t.name == "norm.weight" || t.name == "model.norm.weight") {
            M.norm = &t;
        } else if (t.name == "output.weight" || t.name == "lm_head.weight") {
            M.out = &t;
        }
    }
    if (!M.out)
        M.out = M.emb;   // weight tying (model.c:262-266)
}

// The load plan of one checkpoint: config, mapping, kind of the matrices.
struct Plan {
    Conf c;
    Mapped M;
    int wkind = -1;   // 0 INT8, 1 FP8
};

const char *mat_names[7] = {"wq", "wk", "wv", "wo", "w1", "w2", "w3"};

bool check_matrix(const StFile &F, const StTensor *t, long long rows, long long cols, const std::string &what,
                  int quant_kind, int &wkind, std::string &err)
{
    if (!t) {
        err = "missing tensor: " + what;
        return false;
    }
    if (t->dt == DT_BAD) {
        err = "tensor '" + t->name + "': unsupported dtype";
        return false;
    }
    if (t->shape.size() != 2 || t->shape[0] != rows || t->shape[1] != cols) {
        char b[160];
        snprintf(b, sizeof b, "': shape must be [%lld, %lld]", rows, cols);
        err = "tensor '" + t->name + b;
        return false;
    }
    int kind;
    if (t->dt == DT_I8 || t->dt == DT_F8) {
        kind = t->dt == DT_F8 ? 1 : 0;
        const StTensor *s = F.find(t->name + "_scale");
        if (!s) {
            err = "tensor '" + t->name + "': quantized weights need a scale tensor '" + t->name + "_scale'";
            return false;
        }
        const bool shape_ok = (s->shape.size() == 1 && s->shape[0] == rows) ||
                              (s->shape.size() == 2 && s->shape[0] == rows && s->shape[1] == 1);
        if (s->dt != DT_F32 || !shape_ok) {
            err = "scale tensor '" + s->name + "': must be F32 with one scale per row";
            return false;
        }
    } else {
        kind = quant_kind;
    }
    if (wkind >= 0 && wkind != kind) {
        err = "tensor '" + t->name + "': INT8 and FP8 weights mixed in one model";
        return false;
    }
    wkind = kind;
    return true;
}

bool check_norm(const StTensor *t, long long n, const std::string &what, std::string &err)
{
    if (!t) {
        err = "missing tensor: " + what;
        return false;
    }
    if (!(t->dt == DT_BF16 || t->dt == DT_F16 || t->dt == DT_F32) || t->shape.size() != 1 || t->shape[0] != n) {
        err = "tensor '" + t->name + "': a norm weight must be [dim] BF16, F16 or F32";
        return false;
    }
    return true;
}

bool make_plan(const char *model_path, const char *config_path, int quant_kind, StFile &F, Plan &P,
               std::string &err)
{
    if (!config_path || !load_conf(config_path, P.c, err))
        return err.empty() ? (err = "no config path", false) : false;
    if (!open_st(model_path, F, err))
        return false;
    const Conf &c = P.c;
    map_names(F, c.n_layers, P.M);
    const long long qd = (long long)c.n_heads * c.head_dim, kd = (long long)c.n_kv_heads * c.head_dim;
    const long long shapes[7][2] = {{qd, c.dim}, {kd, c.dim}, {kd, c.dim}, {c.dim, qd},
                                    {c.hidden_dim, c.dim}, {c.dim, c.hidden_dim}, {c.hidden_dim, c.dim}};
    for (int l = 0; l < c.n_layers; l++) {
        for (int m = 0; m < 7; m++)
            if (!check_matrix(F, P.M.L[m][l], shapes[m][0], shapes[m][1],
                              "layers." + std::to_string(l) + "." + mat_names[m], quant_kind, P.wkind, err))
                return false;
        if (!check_norm(P.M.L[M_AN][l], c.dim, "layers." + std::to_string(l) + ".attention_norm", err) ||
            !check_norm(P.M.L[M_FN][l], c.dim, "layers." + std::to_string(l) + ".ffn_norm", err))
            return false;
    }
    if (!check_matrix(F, P.M.emb, c.vocab, c.dim, "token embedding", quant_kind, P.wkind, err) ||
        !check_matrix(F, P.M.out, c.vocab, c.dim, "output", quant_kind, P.wkind, err) ||
        !check_norm(P.M.norm, c.dim, "final norm", err))
        return false;
    return true;
}

float bits_f32(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float f16_to_f32(uint16_t h)
{
    const uint32_t s = (uint32_t)(h & 0x8000) << 16;
    int e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FF;
    if (e == 0x1F)
        return bits_f32(s | 0x7F800000u | (m << 13));
    if (e == 0) {
        if (m == 0)
            return bits_f32(s);
        while (!(m & 0x400)) {   // subnormal: normalise
            m <<= 1;
            e--;
        }
        e++;
        m &= 0x3FF;
    }
    return bits_f32(s | ((uint32_t)(e + 112) << 23) | (m << 13));
}

uint16_t f32_to_bf16_host(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float to_f32(const uint8_t *p, Dt dt)
{
    if (dt == DT_F32) {
        float f;
        memcpy(&f, p, 4);
        return f;
    }
    uint16_t h;
    memcpy(&h, p, 2);
    if (dt == DT_BF16) {
        const uint32_t u = (uint32_t)h << 16;
        float f;
        memcpy(&f, &u, 4);
        return f;
    }
    return f16_to_f32(h);
}

}  // namespace
}  // namespace be42

using namespace be42;

struct be42_model {
    be42_decoder_config cfg{};
    std::vector<void *> dev;            // every device allocation
    std::vector<be42_decoder_layer> layers;
    be42_decoder_weights w{};
    be42_decoder *dec = nullptr;
};

static void model_release(be42_model *m)
{
    if (!m)
        return;
    if (m->dec)
        be42_decoder_destroy(m->dec);
    for (void *p : m->dev)
        (void)hipFree(p);
    delete m;
}

extern "C" void be42_model_free(be42_model *m) { model_release(m); }

extern "C" int be42_model_check(const char *model_path, const char *config_path, int quant_kind,
                                be42_decoder_config *cfg_out, int *wkind_out)
{
    BE42_CHECK(model_path && config_path, "be42_model_check: null path");
    BE42_CHECK(quant_kind == 0 || quant_kind == 1, "be42_model_check: quant_kind %d (0 INT8, 1 FP8)", quant_kind);
    StFile F;
    Plan P;
    std::string err;
    if (!make_plan(model_path, config_path, quant_kind, F, P, err)) {
        set_error("be42_model_check: %s", err.c_str());
        return BE42_EINVAL;
    }
    if (cfg_out) {
        *cfg_out = be42_decoder_config{};
        cfg_out->n_layers = P.c.n_layers;
        cfg_out->dim = P.c.dim;
        cfg_out->n_heads = P.c.n_heads;
        cfg_out->n_kv_heads = P.c.n_kv_heads;
        cfg_out->head_dim = P.c.head_dim;
        cfg_out->hidden_dim = P.c.hidden_dim;
        cfg_out->vocab = P.c.vocab;
        cfg_out->wkind = P.wkind;
        cfg_out->rope_theta = P.c.rope_theta;
        cfg_out->norm_eps = P.c.norm_eps;
    }
    if (wkind_out)
        *wkind_out = P.wkind;
    return BE42_OK;
}

extern "C" int be42_model_load(be42_model **out, const char *model_path, const char *config_path,
                               const be42_model_options *opt)
{
    BE42_CHECK(out && model_path && config_path && opt, "be42_model_load: null pointer");
    *out = nullptr;
    BE42_CHECK(opt->quant_kind == 0 || opt->quant_kind == 1, "be42_model_load: quant_kind %d", opt->quant_kind);
    StFile F;
    Plan P;
    std::string err;
    if (!make_plan(model_path, config_path, opt->quant_kind, F, P, err)) {
        set_error("be42_model_load: %s", err.c_str());
        return BE42_EINVAL;
    }
    be42_model *m = new be42_model();
    const Conf &c = P.c;
    hipError_t e = hipSuccess;
    auto dalloc = [&](size_t bytes) -> void * {
        void *p = nullptr;
        if (e == hipSuccess)
            e = hipMalloc(&p, bytes ? bytes : 4);
        if (e == hipSuccess)
            m->dev.push_back(p);
        return e == hipSuccess ? p : nullptr;
    };
    auto upload = [&](const void *src, size_t bytes) -> void * {
        void *p = dalloc(bytes);
        if (p && e == hipSuccess)
            e = hipMemcpy(p, src, bytes, hipMemcpyHostToDevice);
        return e == hipSuccess ? p : nullptr;
    };
    int rc = BE42_OK;
    // a matrix: codes + per-row scales on the device
    auto matrix = [&](const StTensor *t, const void **codes, const float **scales) {
        if (e != hipSuccess || rc != BE42_OK)
            return;
        const size_t rows = (size_t)t->shape[0], cols = (size_t)t->shape[1];
        if (t->dt == DT_I8 || t->dt == DT_F8) {
            const StTensor *s = F.find(t->name + "_scale");
            *codes = upload(F.data + t->begin, rows * cols);
            *scales = (const float *)upload(F.data + s->begin, rows * 4);
            return;
        }
        // quantize on load, on the device, in slabs of rows
        uint8_t *q = (uint8_t *)dalloc(rows * cols);
        float *sc = (float *)dalloc(rows * 4);
        const size_t slab = std::max<size_t>(1, ((size_t)64 << 20) / (cols * 4));
        std::vector<float> host;
        float *stage = nullptr;
        if (e == hipSuccess)
            e = hipMalloc(&stage, std::min(slab, rows) * cols * 4);
        for (size_t r0 = 0; r0 < rows && e == hipSuccess && rc == BE42_OK; r0 += slab) {
            const size_t nr = std::min(slab, rows - r0);
            host.resize(nr * cols);
            const uint8_t *src = F.data + t->begin + r0 * cols * dt_size(t->dt);
            for (size_t i = 0; i < nr * cols; i++)
                host[i] = to_f32(src + i * dt_size(t->dt), t->dt);
            e = hipMemcpy(stage, host.data(), nr * cols * 4, hipMemcpyHostToDevice);
            if (e == hipSuccess)
                rc = opt->quant_kind == 1
                         ? be42_quant_rows_fp8(q + r0 * cols, sc + r0, stage, (int)nr, (int)cols, nullptr)
                         : be42_quant_rows_int8((int8_t *)q + r0 * cols, sc + r0, stage, (int)nr, (int)cols, nullptr);
            if (e == hipSuccess && rc == BE42_OK)
                e = hipDeviceSynchronize();
        }
        if (stage)
            (void)hipFree(stage);
        *codes = q;
        *scales = sc;
    };
    auto norm = [&](const StTensor *t) -> const uint16_t * {
        std::vector<uint16_t> h((size_t)t->shape[0]);
        for (size_t i = 0; i < h.size(); i++)
            h[i] = t->dt == DT_BF16 ? (uint16_t)(F.data[t->begin + 2 * i] | (F.data[t->begin + 2 * i + 1] << 8))
                                    : f32_to_bf16_host(to_f32(F.data + t->begin + i * dt_size(t->dt), t->dt));
        return (const uint16_t *)upload(h.data(), h.size() * 2);
    };
    m->layers.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        be42_decoder_layer &L = m->layers[l];
        matrix(P.M.L[M_WQ][l], &L.wq, &L.sq);
        matrix(P.M.L[M_WK][l], &L.wk, &L.sk);
        matrix(P.M.L[M_WV][l], &L.wv, &L.sv);
        matrix(P.M.L[M_WO][l], &L.wo, &L.so);
        matrix(P.M.L[M_W1][l], &L.w1, &L.s1);
        matrix(P.M.L[M_W2][l], &L.w2, &L.s2);
        matrix(P.M.L[M_W3][l], &L.w3, &L.s3);
        if (e == hipSuccess && rc == BE42_OK) {
            L.attn_norm = norm(P.M.L[M_AN][l]);
            L.ffn_norm = norm(P.M.L[M_FN][l]);
        }
    }
    matrix(P.M.emb, &m->w.emb, &m->w.emb_s);
    if (P.M.out == P.M.emb) {
        m->w.out = m->w.emb;
        m->w.out_s = m->w.emb_s;
    } else {
        matrix(P.M.out, &m->w.out, &m->w.out_s);
    }
    if (e == hipSuccess && rc == BE42_OK)
        m->w.final_norm = norm(P.M.norm);
    if (e != hipSuccess || rc != BE42_OK) {
        model_release(m);
        return rc != BE42_OK ? rc : hip_fail(e, "be42_model_load", __FILE__, __LINE__);
    }
    m->w.layers = m->layers.data();
    be42_decoder_config &d = m->cfg;
    d.n_layers = c.n_layers;
    d.dim = c.dim;
    d.n_heads = c.n_heads;
    d.n_kv_heads = c.n_kv_heads;
    d.head_dim = c.head_dim;
    d.hidden_dim = c.hidden_dim;
    d.vocab = c.vocab;
    d.max_seq = opt->max_seq > 0 ? opt->max_seq : 8192;   // seq_len 8192 (model.c:140)
    d.max_batch = opt->max_batch > 0 ? opt->max_batch : 1;
    d.wkind = P.wkind;
    d.kv_kind = opt->kv_kind;
    d.sparse_k = opt->sparse_k > 0 ? opt->sparse_k : 64;    // SPARSE_BLOCKS_K (config.h:71-73)
    d.cand_cap = opt->cand_cap > 0 ? opt->cand_cap : 64;
    d.rope_len = opt->rope_len;
    d.rope_theta = c.rope_theta;
    d.norm_eps = c.norm_eps;
    std::vector<float> hp((size_t)16 * c.head_dim), hpT((size_t)16 * c.head_dim);
    be42_lsh_projection(hp.data(), hpT.data(), c.head_dim, opt->lsh_seed > 0 ? (unsigned)opt->lsh_seed : 42u);
    rc = be42_decoder_create(&m->dec, &d, &m->w, hpT.data());
    if (rc != BE42_OK) {
        m->dec = nullptr;
        model_release(m);
        return rc;
    }
    *out = m;
    return BE42_OK;
}

extern "C" be42_decoder *be42_model_decoder(be42_model *m) { return m ? m->dec : nullptr; }

extern "C" int be42_model_config(const be42_model *m, be42_decoder_config *cfg)
{
    BE42_CHECK(m && cfg, "be42_model_config: null pointer");
    *cfg = m->cfg;
    return BE42_OK;
}
