// Sanitizer harness for the host-only parsers of external files (state_dict.cpp, llama2.cpp,
// tokenizer.cpp, bpe.cpp), built with -fsanitize=address,undefined by tests/test_sanitized_parsers.py
// and run on valid, truncated and corrupted files.  A parse error is an ordinary outcome (the call
// returns a status); any out-of-bounds access, overflow or other undefined behaviour aborts the run
// through the sanitizers, which the test reports.
//
// The parsers reference the library's error channel and the model constructors the loaders hand
// tensors to; this harness defines the former and never reaches the latter (they fail if called).
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "ar_hip.h"
#include "ar_llama2.h"
#include "ar_state_dict.h"
#include "ar_tokenizer.h"

static char g_err[1024];
void ar_set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
extern "C" int ar_hip_qwen3_create(ar_hip_ctx*, const ar_qwen3_cfg*, ar_qwen3**) { return AR_HIP_ERR_NO_DEVICE; }
extern "C" int ar_hip_qwen3_destroy(ar_qwen3*) { return AR_HIP_OK; }
extern "C" int ar_hip_qwen3_finalize(ar_qwen3*) { return AR_HIP_ERR_NO_DEVICE; }
extern "C" int ar_hip_qwen3_set_weight(ar_qwen3*, const char*, const void*, int, int64_t) { return AR_HIP_ERR_NO_DEVICE; }

static const char* kTexts[] = {"hello world", "  spaces\tand\nlines  ", "caf\xc3\xa9 \xe6\x97\xa5\xe6\x9c\xac 123",
                               "\xff\xfe broken utf8 \xc3", ""};

static int state_dict(const char* path) {
    ar_state_dict* sd = nullptr;
    if (ar_hip_state_dict_open(path, &sd) != AR_HIP_OK) return 0;
    int n = 0;
    ar_hip_state_dict_size(sd, &n);
    for (int i = 0; i < n; i++) {
        const char* key = nullptr;
        if (ar_hip_state_dict_key(sd, i, &key) != AR_HIP_OK) continue;
        int nd = 0, axis = 0, stored = 0;
        int32_t dims[AR_SD_MAX_DIMS];
        int64_t count = 0;
        if (ar_hip_state_dict_info(sd, key, &nd, dims, &axis, &stored, &count) != AR_HIP_OK || count <= 0 ||
            count > (1 << 24))
            continue;
        std::vector<float> f((size_t)count);
        std::vector<double> d((size_t)count);
        ar_hip_state_dict_read(sd, key, AR_DTYPE_F32, f.data(), count);
        ar_hip_state_dict_read(sd, key, AR_DTYPE_F64, d.data(), count);
    }
    ar_qwen3_cfg cfg;
    ar_hip_qwen3_infer_config(sd, &cfg);
    ar_hip_state_dict_destroy(sd);
    return 0;
}

static int llama2(const char* path) {
    ar_llama2_ckpt* ck = nullptr;
    if (ar_hip_llama2_open(path, &ck) != AR_HIP_OK) return 0;
    static const char* names[] = {"tokenEmbeddings", "rmsAttWeights", "wq", "wk", "wv", "wo", "rmsFfn", "w1",
                                  "w2", "w3", "rmsFinalWeight", "wcls", "freqCis"};
    double sink = 0;
    for (const char* name : names) {
        const float* data = nullptr;
        int64_t n = 0;
        if (ar_hip_llama2_tensor(ck, name, &data, &n) == AR_HIP_OK && n > 0) sink += data[0] + data[n - 1];
    }
    ar_hip_llama2_close(ck);
    return sink == 12345.0 ? 1 : 0;
}

static int bpe(const char* path, int vocab) {
    ar_bpe* t = nullptr;
    if (ar_hip_bpe_load(path, vocab, &t) != AR_HIP_OK) return 0;
    int32_t toks[512];
    for (const char* s : kTexts) {
        int n = 0;
        ar_hip_bpe_encode(t, s, (int)strlen(s), toks, 512, &n);
    }
    int nv = 0;
    ar_hip_bpe_vocab_size(t, &nv);
    for (int i = 0; i < nv; i++) {
        const char* u = nullptr;
        int len = 0;
        float sc = 0;
        ar_hip_bpe_token(t, i, &u, &len, &sc);
    }
    ar_hip_bpe_destroy(t);
    return 0;
}

static int tokenizer(const char* path) {
    ar_tokenizer* t = nullptr;
    if (ar_hip_tokenizer_load(path, &t) != AR_HIP_OK) return 0;
    int32_t ids[1024];
    char out[4096];
    for (const char* s : kTexts) {
        int n = 0;
        if (ar_hip_tokenizer_encode(t, s, (int64_t)strlen(s), 1, 1, ids, 1024, &n) == AR_HIP_OK) {
            int64_t len = 0;
            ar_hip_tokenizer_decode(t, ids, n, out, sizeof out, &len);
        }
    }
    ar_hip_tokenizer_destroy(t);
    return 0;
}

int main(int argc, char** argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: %s statedict|llama2|bpe|tokenizer PATH [VOCAB]\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[1];
    if (mode == "statedict") return state_dict(argv[2]);
    if (mode == "llama2") return llama2(argv[2]);
    if (mode == "bpe") return bpe(argv[2], argc > 3 ? atoi(argv[3]) : 0);
    if (mode == "tokenizer") return tokenizer(argv[2]);
    return 2;
}
