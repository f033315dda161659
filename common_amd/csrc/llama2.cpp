// Llama2 checkpoints (host only): the llama2.c file layout the reference reads with
// TransformerConfig(ByteBuffer) and Llama2Weights (engine/ml/src/main/java/org/almostrealism/ml/
// TransformerConfig.java:69-80, llama2/Llama2Weights.java:90-173), mapped read-only, and the model
// Llama2.model builds from it (llama2/Llama2.java:173-201) as a decoder of include/ar_hip.h.
//
// File layout: seven int32 (dim, hiddenDim, layerCount, headCount, kvHeadCount, vocabSize,
// seqLen), then fp32 tensors back to back in the order Llama2Weights stages them:
//   tokenEmbeddings (V, d)  rmsAttWeights (L, d)  wq wk wv wo (L, d, d)  rmsFfn (L, d)
//   w1 (L, F, d)  w2 (L, d, F)  w3 (L, F, d)  rmsFinalWeight (d)
//   RoPE real plane (S, hs/2)  RoPE imaginary plane (S, hs/2)  [wcls (V, d) when vocabSize < 0]
// The reference reads wk and wv as (d, d) whatever kvHeadCount says and builds heads == kvHeads
// (Llama2.java:181-192); this loader does the same.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <string>
#include <vector>

#include "../../include/ar_llama2.h"

void ar_set_error(const char* fmt, ...);

struct ar_llama2_ckpt {
    ar_llama2_cfg cfg{};
    void* map = nullptr;
    size_t map_bytes = 0;
    const float* base = nullptr;  // first tensor value
    // element offsets from base
    int64_t off_embed = 0, off_rms_att = 0, off_wq = 0, off_wk = 0, off_wv = 0, off_wo = 0, off_rms_ffn = 0,
            off_w1 = 0, off_w2 = 0, off_w3 = 0, off_rms_final = 0, off_freq_re = 0, off_freq_im = 0, off_wcls = 0;
    int64_t end = 0;
    std::vector<float> freq_cis;  // (S, hs/2, 2), the two planes interleaved
};

extern "C" int ar_hip_llama2_parse_config(const void* header, size_t n, ar_llama2_cfg* out) {
    if (!header || !out) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    if (n < AR_LLAMA2_HEADER_BYTES) {
        ar_set_error("checkpoint header needs %d bytes, %zu given", AR_LLAMA2_HEADER_BYTES, n);
        return AR_HIP_ERR_INVALID;
    }
    int32_t v[7];
    memcpy(v, header, sizeof(v));  // little-endian host, as the reference's buffer order
    ar_llama2_cfg c{};
    c.dim = v[0];
    c.hidden_dim = v[1];
    c.layer_count = v[2];
    c.head_count = v[3];
    c.kv_head_count = v[4];
    if (v[5] == INT32_MIN) {
        ar_set_error("checkpoint vocabulary size %d has no absolute value", v[5]);
        return AR_HIP_ERR_INVALID;
    }
    c.vocab_size = v[5] < 0 ? -v[5] : v[5];
    c.seq_len = v[6];
    c.shared_weights = v[5] > 0;
    if (c.head_count == 0) {
        ar_set_error("checkpoint head count is 0");
        return AR_HIP_ERR_INVALID;
    }
    c.head_size = c.dim / c.head_count;
    *out = c;
    return AR_HIP_OK;
}

extern "C" int ar_hip_llama2_close(ar_llama2_ckpt* ck) {
    if (!ck) return AR_HIP_OK;
    if (ck->map) munmap(ck->map, ck->map_bytes);
    delete ck;
    return AR_HIP_OK;
}

extern "C" int ar_hip_llama2_open(const char* path, ar_llama2_ckpt** out) {
    if (!path || !out) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        ar_set_error("cannot open checkpoint '%s': %s", path, strerror(errno));
        return AR_HIP_ERR_NOT_FOUND;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ar_set_error("cannot stat '%s': %s", path, strerror(errno));
        close(fd);
        return AR_HIP_ERR_INVALID;
    }
    const size_t bytes = (size_t)st.st_size;
    if (bytes < AR_LLAMA2_HEADER_BYTES) {
        close(fd);
        ar_set_error("checkpoint '%s' is %zu bytes, shorter than its header", path, bytes);
        return AR_HIP_ERR_INVALID;
    }
    void* map = mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) {
        ar_set_error("cannot map '%s': %s", path, strerror(errno));
        return AR_HIP_ERR_INVALID;
    }
    ar_llama2_ckpt* ck = new ar_llama2_ckpt();
    ck->map = map;
    ck->map_bytes = bytes;
    int rc = ar_hip_llama2_parse_config(map, bytes, &ck->cfg);
    if (rc != AR_HIP_OK) {
        ar_hip_llama2_close(ck);
        return rc;
    }
    const ar_llama2_cfg& c = ck->cfg;
    if (c.dim <= 0 || c.hidden_dim <= 0 || c.layer_count <= 0 || c.head_count <= 0 || c.vocab_size <= 0 ||
        c.seq_len <= 0 || c.dim % c.head_count != 0 || c.head_size % 2 != 0) {
        ar_set_error("checkpoint '%s': bad header (dim %d, hidden %d, layers %d, heads %d, vocab %d, seq %d)", path,
                     c.dim, c.hidden_dim, c.layer_count, c.head_count, c.vocab_size, c.seq_len);
        ar_hip_llama2_close(ck);
        return AR_HIP_ERR_INVALID;
    }
    const int64_t d = c.dim, F = c.hidden_dim, L = c.layer_count, V = c.vocab_size, S = c.seq_len,
                  half = c.head_size / 2;
    // Offsets are sums of products of header fields: every product and sum is checked, so a header
    // whose sizes overflow 64 bits (or describe more floats than the file could hold) is rejected
    // instead of wrapping into a small total that passes the length check below.
    int64_t o = 0;
    bool overflow = false;
    auto prod = [&](std::initializer_list<int64_t> fs) {
        int64_t r = 1;
        for (int64_t f : fs)
            if (__builtin_mul_overflow(r, f, &r)) overflow = true;
        return r;
    };
    auto take = [&](int64_t n) {
        const int64_t at = o;
        if (__builtin_add_overflow(o, n, &o)) overflow = true;
        return at;
    };
    ck->off_embed = take(prod({V, d}));
    ck->off_rms_att = take(prod({L, d}));
    ck->off_wq = take(prod({L, d, d}));
    ck->off_wk = take(prod({L, d, d}));
    ck->off_wv = take(prod({L, d, d}));
    ck->off_wo = take(prod({L, d, d}));
    ck->off_rms_ffn = take(prod({L, d}));
    ck->off_w1 = take(prod({L, F, d}));
    ck->off_w2 = take(prod({L, d, F}));
    ck->off_w3 = take(prod({L, F, d}));
    ck->off_rms_final = take(d);
    ck->off_freq_re = take(prod({S, half}));
    ck->off_freq_im = take(prod({S, half}));
    ck->off_wcls = c.shared_weights ? ck->off_embed : take(prod({V, d}));
    ck->end = o;
    if (overflow || o > (int64_t)((bytes - AR_LLAMA2_HEADER_BYTES) / sizeof(float))) {
        ar_set_error("checkpoint '%s' is %zu bytes; its header describes %s", path, bytes,
                     overflow ? "more than 2^63 floats" : "more floats than the file holds");
        ar_hip_llama2_close(ck);
        return AR_HIP_ERR_INVALID;
    }
    const size_t need = AR_LLAMA2_HEADER_BYTES + (size_t)o * sizeof(float);
    if (bytes < need) {
        ar_set_error("checkpoint '%s' is %zu bytes; its header describes %zu", path, bytes, need);
        ar_hip_llama2_close(ck);
        return AR_HIP_ERR_INVALID;
    }
    ck->base = reinterpret_cast<const float*>(static_cast<const char*>(map) + AR_LLAMA2_HEADER_BYTES);
    // Llama2Weights.stage(shape(S, hs/2, 2), take(re), take(im)): one element from each plane in turn
    ck->freq_cis.resize((size_t)(S * half * 2));
    const float* re = ck->base + ck->off_freq_re;
    const float* im = ck->base + ck->off_freq_im;
    for (int64_t i = 0; i < S * half; i++) {
        ck->freq_cis[(size_t)(2 * i)] = re[i];
        ck->freq_cis[(size_t)(2 * i + 1)] = im[i];
    }
    *out = ck;
    return AR_HIP_OK;
}

extern "C" int ar_hip_llama2_config(const ar_llama2_ckpt* ck, ar_llama2_cfg* out) {
    if (!ck || !out) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *out = ck->cfg;
    return AR_HIP_OK;
}

extern "C" int ar_hip_llama2_tensor(const ar_llama2_ckpt* ck, const char* name, const float** data, int64_t* n) {
    if (!ck || !name || !data || !n) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    const ar_llama2_cfg& c = ck->cfg;
    const int64_t d = c.dim, F = c.hidden_dim, L = c.layer_count, V = c.vocab_size;
    struct Entry {
        const char* name;
        int64_t off, n;
    };
    const Entry table[] = {
        {"tokenEmbeddings", ck->off_embed, V * d}, {"rmsAttWeights", ck->off_rms_att, L * d},
        {"wq", ck->off_wq, L * d * d},             {"wk", ck->off_wk, L * d * d},
        {"wv", ck->off_wv, L * d * d},             {"wo", ck->off_wo, L * d * d},
        {"rmsFfn", ck->off_rms_ffn, L * d},        {"w1", ck->off_w1, L * F * d},
        {"w2", ck->off_w2, L * d * F},             {"w3", ck->off_w3, L * F * d},
        {"rmsFinalWeight", ck->off_rms_final, d},  {"wcls", ck->off_wcls, V * d},
    };
    if (!strcmp(name, "freqCis")) {
        *data = ck->freq_cis.data();
        *n = (int64_t)ck->freq_cis.size();
        return AR_HIP_OK;
    }
    for (const Entry& e : table)
        if (!strcmp(name, e.name)) {
            *data = ck->base + e.off;
            *n = e.n;
            return AR_HIP_OK;
        }
    ar_set_error("no tensor '%s' in a Llama2 checkpoint", name);
    return AR_HIP_ERR_NOT_FOUND;
}

extern "C" int ar_hip_llama2_create_model(ar_hip_ctx* ctx, const ar_llama2_ckpt* ck, int max_batch, int weight_dtype,
                                          int kv_dtype, ar_qwen3** out) {
    if (!ctx || !ck || !out) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *out = nullptr;
    const ar_llama2_cfg& c = ck->cfg;
    ar_qwen3_cfg q{};
    q.dim = c.dim;
    q.hidden_dim = c.hidden_dim;
    q.layer_count = c.layer_count;
    q.head_count = c.head_count;
    q.kv_head_count = c.head_count;  // Llama2.model: transformer(headCount, ...) = heads == kvHeads
    q.head_size = c.head_size;
    q.vocab_size = c.vocab_size;
    q.seq_len = c.seq_len;
    q.max_batch = max_batch;
    q.weight_dtype = weight_dtype;
    q.qk_norm_mode = AR_QK_NORM_WHOLE;  // no QK-norm gains are set: the norm is skipped
    q.shared_weights = c.shared_weights;
    q.qkv_bias = 0;
    q.kv_dtype = kv_dtype;
    q.rope_theta = 10000.0;  // unused: the checkpoint's table replaces the computed one
    q.epsilon = 1e-5;
    ar_qwen3* m = nullptr;
    int rc = ar_hip_qwen3_create(ctx, &q, &m);
    if (rc != AR_HIP_OK) return rc;
    const int64_t d = c.dim, F = c.hidden_dim;
    auto set = [&](const std::string& key, int64_t off, int64_t n) {
        return ar_hip_qwen3_set_weight(m, key.c_str(), ck->base + off, AR_DTYPE_F32, n);
    };
    rc = set("model.embed_tokens.weight", ck->off_embed, (int64_t)c.vocab_size * d);
    if (rc == AR_HIP_OK && !c.shared_weights) rc = set("lm_head.weight", ck->off_wcls, (int64_t)c.vocab_size * d);
    if (rc == AR_HIP_OK) rc = set("model.norm.weight", ck->off_rms_final, d);
    for (int l = 0; rc == AR_HIP_OK && l < c.layer_count; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        const int64_t dd = d * d, fd = F * d;
        rc = set(p + "input_layernorm.weight", ck->off_rms_att + l * d, d);
        if (rc == AR_HIP_OK) rc = set(p + "self_attn.q_proj.weight", ck->off_wq + l * dd, dd);
        if (rc == AR_HIP_OK) rc = set(p + "self_attn.k_proj.weight", ck->off_wk + l * dd, dd);
        if (rc == AR_HIP_OK) rc = set(p + "self_attn.v_proj.weight", ck->off_wv + l * dd, dd);
        if (rc == AR_HIP_OK) rc = set(p + "self_attn.o_proj.weight", ck->off_wo + l * dd, dd);
        if (rc == AR_HIP_OK) rc = set(p + "post_attention_layernorm.weight", ck->off_rms_ffn + l * d, d);
        if (rc == AR_HIP_OK) rc = set(p + "mlp.gate_proj.weight", ck->off_w1 + l * fd, fd);
        if (rc == AR_HIP_OK) rc = set(p + "mlp.down_proj.weight", ck->off_w2 + l * fd, fd);
        if (rc == AR_HIP_OK) rc = set(p + "mlp.up_proj.weight", ck->off_w3 + l * fd, fd);
    }
    if (rc == AR_HIP_OK)
        rc = ar_hip_qwen3_set_weight(m, AR_ROPE_TABLE_KEY, ck->freq_cis.data(), AR_DTYPE_F32,
                                     (int64_t)ck->freq_cis.size());
    if (rc == AR_HIP_OK) rc = ar_hip_qwen3_finalize(m);
    if (rc != AR_HIP_OK) {
        // keep the first error's message: destroying the half-built model sets none
        ar_hip_qwen3_destroy(m);
        return rc;
    }
    *out = m;
    return AR_HIP_OK;
}
