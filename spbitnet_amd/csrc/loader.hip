// loader.hip -- Model::load for the reference's on-disk format
// (docs/compression_format.md:269-439; src/model.cu:72-311): config.json,
// manifest.json and raw little-endian weight files, uploaded to the GPU.
//
// Differences from the reference loader:
//   * the fp16 embedding / LM head is converted to bf16 on the device (the
//     decode engine's storage type); every other tensor keeps its bits;
//   * errors are returned with a message instead of thrown.
// The JSON reader below accepts the subset those two files use (objects,
// arrays, strings with escapes, numbers, true/false/null).
#include <cstdlib>
#include <fstream>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "common.hpp"
#include "spbitnet_amd.h"

namespace spb {
namespace {

struct Json {
    enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;

    const Json* get(const std::string& k) const {
        if (kind != kObj) return nullptr;
        auto it = obj.find(k);
        return it == obj.end() ? nullptr : &it->second;
    }
};

class JsonReader {
  public:
    explicit JsonReader(const std::string& s) : s_(s) {}
    bool parse(Json& out, std::string& err) {
        if (!value(out, 0)) {
            err = err_.empty() ? "malformed JSON" : err_;
            return false;
        }
        ws();
        if (i_ != s_.size()) {
            err = "trailing characters after JSON value";
            return false;
        }
        return true;
    }

  private:
    const std::string& s_;
    size_t i_ = 0;
    std::string err_;

    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t'))
            ++i_;
    }
    bool fail(const char* m) {
        err_ = std::string(m) + " at offset " + std::to_string(i_);
        return false;
    }
    bool lit(const char* w) {
        const size_t n = std::char_traits<char>::length(w);
        if (s_.compare(i_, n, w) != 0) return fail("bad literal");
        i_ += n;
        return true;
    }
    bool string(std::string& out) {
        if (s_[i_] != '"') return fail("expected string");
        ++i_;
        while (i_ < s_.size() && s_[i_] != '"') {
            char c = s_[i_++];
            if (c == '\\') {
                if (i_ >= s_.size()) return fail("bad escape");
                const char e = s_[i_++];
                switch (e) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        if (i_ + 4 > s_.size()) return fail("bad \\u escape");
                        const unsigned cp = static_cast<unsigned>(std::strtoul(s_.substr(i_, 4).c_str(), nullptr, 16));
                        i_ += 4;
                        if (cp < 0x80) {
                            out += static_cast<char>(cp);
                        } else if (cp < 0x800) {
                            out += static_cast<char>(0xC0 | (cp >> 6));
                            out += static_cast<char>(0x80 | (cp & 0x3F));
                        } else {
                            out += static_cast<char>(0xE0 | (cp >> 12));
                            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
                            out += static_cast<char>(0x80 | (cp & 0x3F));
                        }
                        break;
                    }
                    default: return fail("bad escape");
                }
            } else {
                out += c;
            }
        }
        if (i_ >= s_.size()) return fail("unterminated string");
        ++i_;
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (i_ >= s_.size()) return fail("unexpected end");
        const char c = s_[i_];
        if (c == '{') {
            v.kind = Json::kObj;
            ++i_;
            ws();
            if (i_ < s_.size() && s_[i_] == '}') {
                ++i_;
                return true;
            }
            for (;;) {
                ws();
                std::string k;
                if (i_ >= s_.size() || !string(k)) return fail("expected key");
                ws();
                if (i_ >= s_.size() || s_[i_] != ':') return fail("expected ':'");
                ++i_;
                if (!value(v.obj[k], depth + 1)) return false;
                ws();
                if (i_ < s_.size() && s_[i_] == ',') {
                    ++i_;
                    continue;
                }
                if (i_ < s_.size() && s_[i_] == '}') {
                    ++i_;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v.kind = Json::kArr;
            ++i_;
            ws();
            if (i_ < s_.size() && s_[i_] == ']') {
                ++i_;
                return true;
            }
            for (;;) {
                v.arr.emplace_back();
                if (!value(v.arr.back(), depth + 1)) return false;
                ws();
                if (i_ < s_.size() && s_[i_] == ',') {
                    ++i_;
                    continue;
                }
                if (i_ < s_.size() && s_[i_] == ']') {
                    ++i_;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Json::kStr;
            return string(v.str);
        }
        if (c == 't') {
            v.kind = Json::kBool;
            v.b = true;
            return lit("true");
        }
        if (c == 'f') {
            v.kind = Json::kBool;
            return lit("false");
        }
        if (c == 'n') return lit("null");
        const char* start = s_.c_str() + i_;
        char* end = nullptr;
        v.num = std::strtod(start, &end);
        if (end == start) return fail("bad number");
        v.kind = Json::kNum;
        i_ += static_cast<size_t>(end - start);
        return true;
    }
};

bool read_file(const std::string& path, std::string& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    f.seekg(0, std::ios::end);
    const std::streamoff n = f.tellg();
    if (n < 0) return false;
    out.resize(static_cast<size_t>(n));
    f.seekg(0, std::ios::beg);
    return static_cast<bool>(f.read(&out[0], n)) || n == 0;
}

bool read_json(const std::string& path, Json& j, std::string& err) {
    std::string text;
    if (!read_file(path, text)) {
        err = "cannot read " + path;
        return false;
    }
    JsonReader r(text);
    if (!r.parse(j, err)) {
        err = path + ": " + err;
        return false;
    }
    return true;
}

double num_or(const Json& j, const char* k, double dflt) {
    const Json* v = j.get(k);
    return v && v->kind == Json::kNum ? v->num : dflt;
}

// IEEE fp16 bits -> bf16 bits (round to nearest even), on the device.
__global__ void f16_to_bf16_kernel(uint16_t* p, long n) {
    for (long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * 256)
        p[i] = BF16::from_float(F16::to_float(p[i]));
}

}  // namespace
}  // namespace spb

using namespace spb;

struct spb_model {
    spb_model_config cfg{};
    std::vector<spb_transformer_layer> layers;
    std::vector<void*> owned;
    uint16_t* embed = nullptr;
    uint16_t* lm_head = nullptr;
    float* final_norm = nullptr;
    size_t bytes = 0;
    ~spb_model() {
        for (void* p : owned) (void)hipFree(p);
    }
    // Reads `path` (exactly nbytes) into new device memory.
    void* upload(const std::string& path, size_t nbytes, std::string& err) {
        std::string data;
        if (!read_file(path, data)) {
            err = "cannot read " + path;
            return nullptr;
        }
        if (data.size() != nbytes) {
            err = path + ": size " + std::to_string(data.size()) + ", expected " +
                  std::to_string(nbytes);
            return nullptr;
        }
        void* d = nullptr;
        if (hipMalloc(&d, nbytes ? nbytes : 16) != hipSuccess) {
            err = "device allocation failed for " + path;
            return nullptr;
        }
        owned.push_back(d);
        if (nbytes && hipMemcpy(d, data.data(), nbytes, hipMemcpyHostToDevice) != hipSuccess) {
            err = "upload failed for " + path;
            return nullptr;
        }
        bytes += nbytes;
        return d;
    }
};

namespace {

bool load_linear(spb_model* m, const std::string& dir, const Json& e, int rows, int cols,
                 spb_sparse_linear& out, std::string& err) {
    const Json* shape = e.get("shape");
    if (!shape || shape->kind != Json::kArr || shape->arr.size() != 2) {
        err = "sparse entry without a 2-D shape";
        return false;
    }
    out.rows = static_cast<int>(shape->arr[0].num);
    out.cols = static_cast<int>(shape->arr[1].num);
    if (out.rows != rows || out.cols != cols) {
        err = "sparse entry shape " + std::to_string(out.rows) + "x" + std::to_string(out.cols) +
              ", expected " + std::to_string(rows) + "x" + std::to_string(cols);
        return false;
    }
    // meta_stride, values_stride and gamma are required, as in the
    // reference (src/model.cu:107-109 reads them with entry.at()), and the
    // strides must cover a row (ceil(cols/32) meta and ceil(cols/64) sign
    // words): an understated stride would make every kernel read past its row.
    for (const char* key : {"meta_stride", "values_stride", "gamma"}) {
        const Json* v = e.get(key);
        if (!v || v->kind != Json::kNum) {
            err = std::string("sparse entry without numeric ") + key;
            return false;
        }
    }
    out.meta_stride = static_cast<int>(e.get("meta_stride")->num);
    out.values_stride = static_cast<int>(e.get("values_stride")->num);
    out.gamma = static_cast<float>(e.get("gamma")->num);
    if (out.meta_stride < (cols + 31) / 32 || out.values_stride < (cols + 63) / 64) {
        err = "sparse entry strides " + std::to_string(out.meta_stride) + "/" +
              std::to_string(out.values_stride) + " do not cover a row of " +
              std::to_string(cols) + " columns";
        return false;
    }
    const Json* mf = e.get("meta_file");
    const Json* vf = e.get("values_file");
    if (!mf || !vf || mf->kind != Json::kStr || vf->kind != Json::kStr) {
        err = "sparse entry without meta_file / values_file";
        return false;
    }
    out.meta = static_cast<const uint32_t*>(
        m->upload(dir + "/" + mf->str, static_cast<size_t>(out.rows) * out.meta_stride * 4, err));
    if (!out.meta) return false;
    out.values = static_cast<const uint32_t*>(m->upload(
        dir + "/" + vf->str, static_cast<size_t>(out.rows) * out.values_stride * 4, err));
    return out.values != nullptr;
}

const float* load_f32(spb_model* m, const std::string& dir, const Json* weights,
                      const std::string& name, size_t n, std::string& err, bool& present) {
    present = false;
    const Json* e = weights->get(name);
    if (!e) return nullptr;
    present = true;
    const Json* f = e->get("file");
    if (!f || f->kind != Json::kStr) {
        err = name + ": entry without file";
        return nullptr;
    }
    return static_cast<const float*>(m->upload(dir + "/" + f->str, n * 4, err));
}

uint16_t* load_f16_as_bf16(spb_model* m, const std::string& dir, const Json& e, size_t n,
                           std::string& err) {
    const Json* f = e.get("file");
    if (!f || f->kind != Json::kStr) {
        err = "16-bit entry without file";
        return nullptr;
    }
    uint16_t* d = static_cast<uint16_t*>(m->upload(dir + "/" + f->str, n * 2, err));
    if (!d) return nullptr;
    const Json* dt = e.get("dtype");
    if (!dt || dt->str != "bfloat16") {  // the reference writes float16
        long blocks = static_cast<long>((n + 255) / 256);
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(f16_to_bf16_kernel, dim3(blocks), dim3(256), 0, 0, d,
                           static_cast<long>(n));
        if (hipDeviceSynchronize() != hipSuccess) {
            err = "fp16 -> bf16 conversion failed";
            return nullptr;
        }
    }
    return d;
}

}  // namespace

extern "C" int spb_model_load(const char* model_dir, spb_model** out) {
    clear_error();
    const char* fn = "spb_model_load";
    if (!model_dir || !out) return invalid("%s: null argument", fn);
    *out = nullptr;
    const std::string dir(model_dir);
    std::string err;
    Json cj, mj;
    if (!read_json(dir + "/config.json", cj, err) || !read_json(dir + "/manifest.json", mj, err))
        return invalid("%s: %s", fn, err.c_str());
    std::unique_ptr<spb_model> m(new (std::nothrow) spb_model());
    if (!m) return invalid("%s: out of host memory", fn);
    // config.json (src/model.cu:72-89): required fields and the reference's defaults
    spb_model_config& c = m->cfg;
    const char* req[] = {"hidden_size", "num_hidden_layers", "num_attention_heads",
                         "intermediate_size", "vocab_size", "max_position_embeddings"};
    for (const char* k : req)
        if (!cj.get(k)) return invalid("%s: config.json lacks %s", fn, k);
    c.hidden_size = static_cast<int>(num_or(cj, "hidden_size", 0));
    c.num_hidden_layers = static_cast<int>(num_or(cj, "num_hidden_layers", 0));
    c.num_attention_heads = static_cast<int>(num_or(cj, "num_attention_heads", 0));
    c.num_key_value_heads = static_cast<int>(num_or(cj, "num_key_value_heads", c.num_attention_heads));
    c.intermediate_size = static_cast<int>(num_or(cj, "intermediate_size", 0));
    c.vocab_size = static_cast<int>(num_or(cj, "vocab_size", 0));
    c.max_position_embeddings = static_cast<int>(num_or(cj, "max_position_embeddings", 0));
    c.rms_norm_eps = static_cast<float>(num_or(cj, "rms_norm_eps", 1e-5));
    c.rope_theta = static_cast<float>(num_or(cj, "rope_theta", 10000.0));
    c.head_dim = static_cast<int>(
        num_or(cj, "head_dim", c.num_attention_heads ? c.hidden_size / c.num_attention_heads : 0));
    c.bos_token_id = static_cast<int>(num_or(cj, "bos_token_id", 1));
    c.eos_token_id = static_cast<int>(num_or(cj, "eos_token_id", 2));
    if (c.hidden_size <= 0 || c.num_hidden_layers <= 0 || c.num_attention_heads <= 0 ||
        c.num_key_value_heads <= 0 || c.intermediate_size <= 0 || c.vocab_size <= 0)
        return invalid("%s: non-positive dimension in config.json", fn);
    const Json* w = mj.get("weights");
    if (!w || w->kind != Json::kObj) return invalid("%s: manifest.json lacks \"weights\"", fn);
    const int H = c.hidden_size, I = c.intermediate_size;
    const int kvd = c.num_key_value_heads * c.head_dim;
    const size_t vh = static_cast<size_t>(c.vocab_size) * H;
    const Json* emb = w->get("embed_tokens");
    if (!emb) return invalid("%s: manifest has no embed_tokens", fn);
    if (!(m->embed = load_f16_as_bf16(m.get(), dir, *emb, vh, err)))
        return invalid("%s: embed_tokens: %s", fn, err.c_str());
    bool present = false;
    m->final_norm = const_cast<float*>(load_f32(m.get(), dir, w, "norm", H, err, present));
    if (!m->final_norm) return invalid("%s: norm: %s", fn, present ? err.c_str() : "missing");
    const Json* lm = w->get("lm_head");
    if (lm && !(lm->get("dtype") && lm->get("dtype")->str == "tied")) {
        if (!(m->lm_head = load_f16_as_bf16(m.get(), dir, *lm, vh, err)))
            return invalid("%s: lm_head: %s", fn, err.c_str());
    }
    m->layers.resize(c.num_hidden_layers);
    for (int l = 0; l < c.num_hidden_layers; ++l) {
        spb_transformer_layer& L = m->layers[l];
        const std::string p = "layers." + std::to_string(l);
        struct Proj {
            const char* name;
            spb_sparse_linear* dst;
            int rows, cols;
        } projs[] = {{"self_attn.q_proj", &L.q_proj, H, H},
                     {"self_attn.k_proj", &L.k_proj, kvd, H},
                     {"self_attn.v_proj", &L.v_proj, kvd, H},
                     {"self_attn.o_proj", &L.o_proj, H, H},
                     {"mlp.gate_proj", &L.gate_proj, I, H},
                     {"mlp.up_proj", &L.up_proj, I, H},
                     {"mlp.down_proj", &L.down_proj, H, I}};
        for (const Proj& pr : projs) {
            const std::string name = p + "." + pr.name;
            const Json* e = w->get(name);
            if (!e) return invalid("%s: manifest lacks %s", fn, name.c_str());
            if (!load_linear(m.get(), dir, *e, pr.rows, pr.cols, *pr.dst, err))
                return invalid("%s: %s: %s", fn, name.c_str(), err.c_str());
        }
        struct Norm {
            const char* name;
            const float** dst;
            int n;
            bool required;
        } norms[] = {{"input_layernorm", &L.input_layernorm, H, true},
                     {"post_attention_layernorm", &L.post_attention_layernorm, H, true},
                     {"self_attn.attn_sub_norm", &L.attn_sub_norm, H, false},
                     {"mlp.ffn_sub_norm", &L.ffn_sub_norm, I, false}};
        for (const Norm& nm : norms) {
            const std::string name = p + "." + nm.name;
            *nm.dst = load_f32(m.get(), dir, w, name, static_cast<size_t>(nm.n), err, present);
            if (!*nm.dst && (present || nm.required))
                return invalid("%s: %s: %s", fn, name.c_str(), present ? err.c_str() : "missing");
        }
    }
    *out = m.release();
    return 0;
}

extern "C" int spb_model_destroy(spb_model* m) {
    clear_error();
    delete m;
    return 0;
}

extern "C" int spb_model_info(const spb_model* m, spb_model_config* cfg,
                              const spb_transformer_layer** layers,
                              const uint16_t** embed_tokens, const uint16_t** lm_head,
                              const float** final_norm, size_t* gpu_bytes) {
    clear_error();
    if (!m) return invalid("spb_model_info: null model");
    if (cfg) *cfg = m->cfg;
    if (layers) *layers = m->layers.data();
    if (embed_tokens) *embed_tokens = m->embed;
    if (lm_head) *lm_head = m->lm_head;
    if (final_norm) *final_norm = m->final_norm;
    if (gpu_bytes) *gpu_bytes = m->bytes;
    return 0;
}
