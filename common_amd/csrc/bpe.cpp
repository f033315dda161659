// Score-driven BPE of llama2.c tokenizers (host only): the tokenizer.bin read of the Llama2
// constructor (engine/ml/src/main/java/org/almostrealism/ml/llama2/Llama2.java:130-146) and
// BPE.lookup / BPE.encode (engine/ml/src/main/java/org/almostrealism/ml/BPE.java:33-101).
//
// Strings are compared as Java compares them, by UTF-16 code units: each vocabulary entry is its
// bytes decoded as UTF-8 with U+FFFD replacing malformed input, and encoding starts from one token
// per UTF-16 unit of the text (a supplementary character is two units, neither of which can equal
// a decoded entry, so such text is rejected as the reference rejects it).  lookup returns the first
// id holding a string, as the reference's linear scan does, through a hash map filled in id order.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ar_llama2.h"
#include "utf8.h"

void ar_set_error(const char* fmt, ...);

struct ar_bpe {
    std::vector<std::string> utf8;      // vocab[i] re-encoded as UTF-8
    std::vector<std::u16string> units;  // vocab[i] as Java holds it
    std::vector<float> scores;
    std::unordered_map<std::u16string, int> first;  // string -> lowest id
};

namespace {

std::u16string to_units(const std::vector<uint32_t>& cps) {
    std::u16string s;
    s.reserve(cps.size());
    for (uint32_t cp : cps) {
        if (cp < 0x10000) {
            s.push_back((char16_t)cp);
        } else {
            cp -= 0x10000;
            s.push_back((char16_t)(0xD800 + (cp >> 10)));
            s.push_back((char16_t)(0xDC00 + (cp & 0x3FF)));
        }
    }
    return s;
}

void add_entry(ar_bpe* t, const unsigned char* bytes, size_t len, float score) {
    std::string s = utf8::utf8_sanitize(bytes, len);
    std::vector<uint32_t> cps;
    std::vector<size_t> offs;
    utf8::utf8_decode(s.data(), s.size(), &cps, &offs);  // valid after sanitising
    std::u16string u = to_units(cps);
    t->first.emplace(u, (int)t->units.size());  // keeps the lowest id of a repeated string
    t->utf8.push_back(std::move(s));
    t->units.push_back(std::move(u));
    t->scores.push_back(score);
}

int lookup_units(const ar_bpe* t, const std::u16string& s) {
    auto it = t->first.find(s);
    return it == t->first.end() ? -1 : it->second;
}

}  // namespace

extern "C" int ar_hip_bpe_load(const char* path, int vocab_size, ar_bpe** out) {
    if (!path || !out) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *out = nullptr;
    if (vocab_size < 0) {
        ar_set_error("negative vocabulary size %d", vocab_size);
        return AR_HIP_ERR_INVALID;
    }
    FILE* f = fopen(path, "rb");
    if (!f) {
        ar_set_error("cannot open tokenizer '%s': %s", path, strerror(errno));
        return AR_HIP_ERR_NOT_FOUND;
    }
    std::vector<unsigned char> data;
    unsigned char buf[1 << 16];
    size_t got;
    while ((got = fread(buf, 1, sizeof(buf), f)) > 0) data.insert(data.end(), buf, buf + got);
    const bool err = ferror(f) != 0;
    fclose(f);
    if (err) {
        ar_set_error("cannot read tokenizer '%s'", path);
        return AR_HIP_ERR_INVALID;
    }
    size_t pos = 0;
    auto need = [&](size_t n) { return data.size() - pos >= n; };
    if (!need(4)) {
        ar_set_error("tokenizer '%s' ends before its max token length", path);
        return AR_HIP_ERR_INVALID;
    }
    pos += 4;  // max token length: not used
    ar_bpe* t = new ar_bpe();
    t->utf8.reserve((size_t)vocab_size);
    t->units.reserve((size_t)vocab_size);
    t->scores.reserve((size_t)vocab_size);
    for (int i = 0; i < vocab_size; i++) {
        float score;
        int32_t len;
        if (!need(8)) {
            ar_set_error("tokenizer '%s' ends at entry %d of %d", path, i, vocab_size);
            delete t;
            return AR_HIP_ERR_INVALID;
        }
        memcpy(&score, data.data() + pos, 4);
        memcpy(&len, data.data() + pos + 4, 4);
        pos += 8;
        if (len < 0 || !need((size_t)len)) {
            ar_set_error("tokenizer '%s': entry %d has length %d past the end of the file", path, i, len);
            delete t;
            return AR_HIP_ERR_INVALID;
        }
        add_entry(t, data.data() + pos, (size_t)len, score);
        pos += (size_t)len;
    }
    *out = t;
    return AR_HIP_OK;
}

extern "C" int ar_hip_bpe_create(const char* const* vocab, const float* scores, int n, ar_bpe** out) {
    if (!out || n < 0 || (n > 0 && (!vocab || !scores))) {
        ar_set_error("bad argument");
        return AR_HIP_ERR_INVALID;
    }
    *out = nullptr;
    ar_bpe* t = new ar_bpe();
    for (int i = 0; i < n; i++) {
        if (!vocab[i]) {
            ar_set_error("vocabulary entry %d is null", i);
            delete t;
            return AR_HIP_ERR_INVALID;
        }
        add_entry(t, (const unsigned char*)vocab[i], strlen(vocab[i]), scores[i]);
    }
    *out = t;
    return AR_HIP_OK;
}

extern "C" int ar_hip_bpe_destroy(ar_bpe* t) {
    delete t;
    return AR_HIP_OK;
}

extern "C" int ar_hip_bpe_vocab_size(const ar_bpe* t, int* n) {
    if (!t || !n) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *n = (int)t->units.size();
    return AR_HIP_OK;
}

extern "C" int ar_hip_bpe_token(const ar_bpe* t, int id, const char** s, int* len, float* score) {
    if (!t || !s || !len) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    if (id < 0 || id >= (int)t->units.size()) {
        ar_set_error("token %d outside the vocabulary of %zu", id, t->units.size());
        return AR_HIP_ERR_INVALID;
    }
    *s = t->utf8[(size_t)id].data();
    *len = (int)t->utf8[(size_t)id].size();
    if (score) *score = t->scores[(size_t)id];
    return AR_HIP_OK;
}

extern "C" int ar_hip_bpe_lookup(const ar_bpe* t, const char* text, int len, int* id) {
    if (!t || !id || (len > 0 && !text) || len < 0) {
        ar_set_error("bad argument");
        return AR_HIP_ERR_INVALID;
    }
    std::vector<uint32_t> cps;
    std::vector<size_t> offs;
    if (!utf8::utf8_decode(text, (size_t)len, &cps, &offs)) {
        ar_set_error("text is not valid UTF-8");
        return AR_HIP_ERR_INVALID;
    }
    *id = lookup_units(t, to_units(cps));
    return AR_HIP_OK;
}

extern "C" int ar_hip_bpe_encode(const ar_bpe* t, const char* text, int len, int32_t* tokens, int cap, int* n) {
    if (!t || !n || len < 0 || (len > 0 && !text) || cap < 0 || (cap > 0 && !tokens)) {
        ar_set_error("bad argument");
        return AR_HIP_ERR_INVALID;
    }
    *n = 0;
    std::vector<uint32_t> cps;
    std::vector<size_t> offs;
    if (!utf8::utf8_decode(text, (size_t)len, &cps, &offs)) {
        ar_set_error("text is not valid UTF-8");
        return AR_HIP_ERR_INVALID;
    }
    const std::u16string units = to_units(cps);
    if (units.size() > (size_t)cap) {
        ar_set_error("text of %zu UTF-16 units exceeds the %d-token buffer", units.size(), cap);
        return AR_HIP_ERR_INVALID;
    }
    std::vector<int> tok;
    tok.reserve(units.size());
    for (size_t i = 0; i < units.size(); i++) {
        const int id = lookup_units(t, std::u16string(1, units[i]));
        if (id < 0) {
            ar_set_error("character U+%04X at UTF-16 index %zu has no token", (unsigned)units[i], i);
            return AR_HIP_ERR_INVALID;
        }
        tok.push_back(id);
    }
    // merge the best-scoring adjacent pair until none concatenates to a token
    std::u16string pair;
    for (;;) {
        float best_score = -1e10f;
        int best_id = -1;
        size_t best_at = 0;
        for (size_t i = 0; i + 1 < tok.size(); i++) {
            pair = t->units[(size_t)tok[i]];
            pair += t->units[(size_t)tok[i + 1]];
            const int id = lookup_units(t, pair);
            if (id != -1 && t->scores[(size_t)id] > best_score) {
                best_score = t->scores[(size_t)id];
                best_id = id;
                best_at = i;
            }
        }
        if (best_id == -1) break;
        tok[best_at] = best_id;
        tok.erase(tok.begin() + (ptrdiff_t)best_at + 1);
    }
    for (size_t i = 0; i < tok.size(); i++) tokens[i] = tok[i];
    *n = (int)tok.size();
    return AR_HIP_OK;
}
