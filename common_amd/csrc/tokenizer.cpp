// Qwen3 byte-level BPE tokenizer (host only): Qwen3Tokenizer over ByteLevelBPETokenizer,
// RegexPreTokenizer and ByteLevelEncoder (engine/ml/src/main/java/org/almostrealism/ml/qwen3/
// Qwen3Tokenizer.java, engine/ml/src/main/java/org/almostrealism/ml/tokenization/).
//
// Pre-tokenisation.  The reference splits text with java.util.regex and the pattern
// (RegexPreTokenizer.java:89-98)
//     's|'t|'re|'ve|'m|'ll|'d | [^\r\n\p{L}\p{N}]?\p{L}+ | \p{N} | ?[^\s\p{L}\p{N}]+[\r\n]*
//     | \s*[\r\n]+ | \s+(?!\S) | \s+
// where \s is Java's ASCII whitespace [ \t\n\x0B\f\r] and \p{L} / \p{N} are the Unicode 13
// letter / number categories (unicode_tables.h).  Matching it leftmost-first with backtracking
// reduces to a scanner: at each position the first alternative that can match decides, with
//   - the optional one-character prefix of the letter run taken when a letter follows it;
//   - the optional space of the punctuation run taken when punctuation follows it;
//   - \s*[\r\n]+ ending after the last CR/LF of the whitespace run (the greedy \s* gives back
//     characters until a CR/LF follows);
//   - \s+(?!\S) taking the whitespace run minus its last character when non-whitespace follows
//     (the whole run at the end of the text; nothing for a single character).
// Every character matches some alternative, so no text is dropped.
//
// Byte-level mapping (ByteLevelEncoder.java): bytes '!'..'~', 0xA1..0xAC and 0xAE..0xFF map to the
// code point of the same value, the other 68 bytes to U+0100 upwards in byte order.
//
// BPE (ByteLevelBPETokenizer.applyBPEMerges): repeatedly merge the one adjacent pair with the
// lowest priority number (the leftmost on ties) until no pair has a merge.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ar_tokenizer.h"
#include "unicode_tables.h"
#include "utf8.h"

using utf8::put_utf8;
using utf8::utf8_decode;
using utf8::utf8_sanitize;

void ar_set_error(const char* fmt, ...);

namespace {

template <size_t N>
bool in_ranges(const UnicodeRange (&r)[N], uint32_t cp) {
    size_t lo = 0, hi = N;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (cp < r[mid].lo)
            hi = mid;
        else if (cp > r[mid].hi)
            lo = mid + 1;
        else
            return true;
    }
    return false;
}

bool is_letter(uint32_t c) { return in_ranges(kLetterRanges, c); }
bool is_number(uint32_t c) { return in_ranges(kNumberRanges, c); }
bool is_space(uint32_t c) { return c == ' ' || c == '\t' || c == '\n' || c == 0x0B || c == '\f' || c == '\r'; }
bool is_crlf(uint32_t c) { return c == '\r' || c == '\n'; }
bool is_punct(uint32_t c) { return !is_space(c) && !is_letter(c) && !is_number(c); }

// End (exclusive, in code points) of the pattern match at i; i when nothing matches.
size_t match_at(const std::vector<uint32_t>& c, size_t i) {
    const size_t n = c.size();
    auto at = [&](size_t k) -> uint32_t { return k < n ? c[k] : 0xFFFFFFFFu; };
    const uint32_t c0 = c[i];
    // 's|'t|'re|'ve|'m|'ll|'d
    if (c0 == '\'') {
        const uint32_t a = at(i + 1), b = at(i + 2);
        if (a == 's' || a == 't') return i + 2;
        if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e')) return i + 3;
        if (a == 'm') return i + 2;
        if (a == 'l' && b == 'l') return i + 3;
        if (a == 'd') return i + 2;
    }
    // [^\r\n\p{L}\p{N}]?\p{L}+
    {
        size_t j = i;
        if (!is_crlf(c0) && !is_letter(c0) && !is_number(c0) && i + 1 < n && is_letter(c[i + 1]))
            j = i + 1;
        if (is_letter(c[j])) {
            while (j < n && is_letter(c[j])) j++;
            return j;
        }
    }
    // \p{N}
    if (is_number(c0)) return i + 1;
    // ' ?[^\s\p{L}\p{N}]+[\r\n]*'
    {
        size_t j = i;
        if (c0 == ' ' && i + 1 < n && is_punct(c[i + 1])) j = i + 1;
        if (j < n && is_punct(c[j])) {
            while (j < n && is_punct(c[j])) j++;
            while (j < n && is_crlf(c[j])) j++;
            return j;
        }
    }
    if (is_space(c0)) {
        size_t e = i;
        while (e < n && is_space(c[e])) e++;
        // \s*[\r\n]+
        for (size_t p = e; p > i; p--)
            if (is_crlf(c[p - 1])) return p;
        // \s+(?!\S)
        if (e == n) return e;
        if (e - i >= 2) return e - 1;
        // \s+
        return e;
    }
    return i;
}

void pretokenize(const std::vector<uint32_t>& c, std::vector<std::pair<size_t, size_t>>* segs) {
    size_t i = 0;
    while (i < c.size()) {
        const size_t j = match_at(c, i);
        if (j > i) {
            segs->emplace_back(i, j);
            i = j;
        } else {
            i++;  // Matcher.find moves on (cannot happen with this pattern)
        }
    }
}

struct ByteMap {
    uint32_t to_cp[256];
    int from_cp[512];  // byte of a mapped code point (< 0x200), -1 otherwise
    ByteMap() {
        std::fill(from_cp, from_cp + 512, -1);
        int n = 0;
        for (int b = 0; b < 256; b++) {
            const bool same = (b >= '!' && b <= '~') || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
            to_cp[b] = same ? (uint32_t)b : (uint32_t)(256 + n++);
            from_cp[to_cp[b]] = b;
        }
    }
};
const ByteMap& byte_map() {
    static const ByteMap m;
    return m;
}

struct Merge {
    std::string merged;
    int priority;
};

}  // namespace

struct ar_tokenizer {
    std::vector<std::string> vocab;  // UTF-8
    std::vector<float> scores;
    std::unordered_map<std::string, int> ids;
    std::unordered_map<std::string, Merge> merges;  // "first second" -> merged, priority
};

namespace {

bool is_special(int id) {
    return id == AR_QWEN3_BOS_TOKEN || id == AR_QWEN3_EOS_TOKEN || id == AR_QWEN3_UNK_TOKEN;  // PAD == BOS
}

std::vector<std::string> bpe(const ar_tokenizer* t, std::vector<std::string> tokens) {
    if (tokens.size() <= 1 || t->merges.empty()) return tokens;
    std::string pair;
    while (true) {
        int best = -1, best_pri = INT_MAX;
        const std::string* best_merged = nullptr;
        for (size_t i = 0; i + 1 < tokens.size(); i++) {
            pair.assign(tokens[i]);
            pair += ' ';
            pair += tokens[i + 1];
            auto it = t->merges.find(pair);
            if (it != t->merges.end() && it->second.priority < best_pri) {
                best_pri = it->second.priority;
                best = (int)i;
                best_merged = &it->second.merged;
            }
        }
        if (best < 0) break;
        tokens[best] = *best_merged;
        tokens.erase(tokens.begin() + best + 1);
    }
    return tokens;
}

int parse_merges(ar_tokenizer* t, const char* path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) {
        ar_set_error("cannot open merges file '%s'", path);
        return AR_HIP_ERR_NOT_FOUND;
    }
    std::string data((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    const std::string text = utf8_sanitize((const unsigned char*)data.data(), data.size());
    int priority = 0;
    size_t i = 0;
    while (i < text.size()) {
        // BufferedReader.readLine: a line ends at \n, \r or \r\n
        size_t e = i;
        while (e < text.size() && text[e] != '\n' && text[e] != '\r') e++;
        const std::string line = text.substr(i, e - i);
        if (e < text.size() && text[e] == '\r' && e + 1 < text.size() && text[e + 1] == '\n')
            i = e + 2;
        else
            i = e + 1;
        // String.trim: code points <= U+0020 at both ends
        size_t a = 0, b = line.size();
        while (a < b && (unsigned char)line[a] <= 0x20) a++;
        while (b > a && (unsigned char)line[b - 1] <= 0x20) b--;
        if ((!line.empty() && line[0] == '#') || a == b) continue;
        const size_t sp = line.find(' ');
        if (sp == std::string::npos) continue;  // split(" ", 2) gives one part
        const std::string first = line.substr(0, sp), second = line.substr(sp + 1);
        const std::string merged = first + second;
        if (!t->ids.count(first) || !t->ids.count(second) || !t->ids.count(merged)) {
            priority++;
            continue;
        }
        t->merges[first + " " + second] = Merge{merged, priority};
        priority++;
    }
    return AR_HIP_OK;
}

}  // namespace

extern "C" int ar_hip_tokenizer_load(const char* tokenizer_path, ar_tokenizer** out) {
    if (!tokenizer_path || !out) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *out = nullptr;
    std::ifstream f(tokenizer_path, std::ios::binary);
    if (!f) {
        ar_set_error("cannot open tokenizer '%s': %s", tokenizer_path, strerror(errno));
        return AR_HIP_ERR_NOT_FOUND;
    }
    std::string data((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    size_t pos = 0;
    auto need = [&](size_t k) { return pos + k <= data.size(); };
    auto rd_i32 = [&]() {
        int32_t v;
        std::memcpy(&v, data.data() + pos, 4);
        pos += 4;
        return v;
    };
    if (!need(4)) {
        ar_set_error("tokenizer '%s' is truncated", tokenizer_path);
        return AR_HIP_ERR_INVALID;
    }
    const int32_t n = rd_i32();
    if (n < 0) {
        ar_set_error("tokenizer '%s': vocabulary size %d", tokenizer_path, n);
        return AR_HIP_ERR_INVALID;
    }
    auto t = std::make_unique<ar_tokenizer>();
    t->vocab.resize((size_t)n);
    t->scores.resize((size_t)n);
    t->ids.reserve((size_t)n);
    for (int32_t i = 0; i < n; i++) {
        if (!need(8)) {
            ar_set_error("tokenizer '%s' is truncated at token %d", tokenizer_path, i);
            return AR_HIP_ERR_INVALID;
        }
        std::memcpy(&t->scores[i], data.data() + pos, 4);
        pos += 4;
        const int32_t len = rd_i32();
        if (len < 0 || !need((size_t)len)) {
            ar_set_error("tokenizer '%s' is truncated at token %d", tokenizer_path, i);
            return AR_HIP_ERR_INVALID;
        }
        t->vocab[i] = utf8_sanitize((const unsigned char*)data.data() + pos, (size_t)len);
        pos += (size_t)len;
        t->ids[t->vocab[i]] = i;
    }
    // merges.txt in the tokenizer's directory (Path.getParent: none for a bare file name)
    const std::string p(tokenizer_path);
    const size_t slash = p.rfind('/');
    if (slash != std::string::npos) {
        const std::string mp = p.substr(0, slash + 1) + "merges.txt";
        struct stat st;
        if (stat(mp.c_str(), &st) == 0) {
            const int rc = parse_merges(t.get(), mp.c_str());
            if (rc != AR_HIP_OK) return rc;
        }
    }
    *out = t.release();
    return AR_HIP_OK;
}

extern "C" int ar_hip_tokenizer_from_vocab(const char* const* vocab, const int32_t* lens, const float* scores, int n,
                                           ar_tokenizer** out) {
    if (!out || (n > 0 && !vocab) || n < 0) {
        ar_set_error("bad argument");
        return AR_HIP_ERR_INVALID;
    }
    auto t = std::make_unique<ar_tokenizer>();
    t->vocab.resize((size_t)n);
    t->scores.assign((size_t)n, 0.f);
    for (int i = 0; i < n; i++) {
        if (!vocab[i]) {
            ar_set_error("vocabulary entry %d is null", i);
            return AR_HIP_ERR_INVALID;
        }
        const size_t len = lens ? (size_t)lens[i] : strlen(vocab[i]);
        t->vocab[i] = utf8_sanitize((const unsigned char*)vocab[i], len);
        if (scores) t->scores[i] = scores[i];
        t->ids[t->vocab[i]] = i;
    }
    *out = t.release();
    return AR_HIP_OK;
}

extern "C" int ar_hip_tokenizer_load_merges(ar_tokenizer* t, const char* merges_path) {
    if (!t || !merges_path) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    return parse_merges(t, merges_path);
}

extern "C" int ar_hip_tokenizer_destroy(ar_tokenizer* t) {
    delete t;
    return AR_HIP_OK;
}

extern "C" int ar_hip_tokenizer_vocab_size(const ar_tokenizer* t, int* n) {
    if (!t || !n) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *n = (int)t->vocab.size();
    return AR_HIP_OK;
}

extern "C" int ar_hip_tokenizer_merge_count(const ar_tokenizer* t, int* n) {
    if (!t || !n) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    *n = (int)t->merges.size();
    return AR_HIP_OK;
}

extern "C" int ar_hip_tokenizer_token(const ar_tokenizer* t, int id, const char** utf8, int* len, float* score) {
    if (!t || !utf8 || !len) {
        ar_set_error("null argument");
        return AR_HIP_ERR_INVALID;
    }
    if (id < 0 || id >= (int)t->vocab.size()) {
        ar_set_error("token id %d outside 0..%d", id, (int)t->vocab.size() - 1);
        return AR_HIP_ERR_INVALID;
    }
    *utf8 = t->vocab[id].c_str();
    *len = (int)t->vocab[id].size();
    if (score) *score = t->scores[id];
    return AR_HIP_OK;
}

extern "C" int ar_hip_tokenizer_pretokenize(const char* text, int64_t text_len, int64_t* offsets, int capacity,
                                            int* count) {
    if ((!text && text_len) || !count || text_len < 0) {
        ar_set_error("bad argument");
        return AR_HIP_ERR_INVALID;
    }
    std::vector<uint32_t> cps;
    std::vector<size_t> offs;
    if (!utf8_decode(text, (size_t)text_len, &cps, &offs)) {
        ar_set_error("text is not valid UTF-8");
        return AR_HIP_ERR_INVALID;
    }
    std::vector<std::pair<size_t, size_t>> segs;
    pretokenize(cps, &segs);
    *count = (int)segs.size();
    if (offsets)
        for (int k = 0; k < (int)segs.size() && k < capacity; k++) {
            offsets[2 * k] = (int64_t)offs[segs[k].first];
            offsets[2 * k + 1] = (int64_t)offs[segs[k].second];
        }
    if ((int)segs.size() > capacity && offsets) {
        ar_set_error("%d segments for room of %d", (int)segs.size(), capacity);
        return AR_HIP_ERR_INVALID;
    }
    return AR_HIP_OK;
}

extern "C" int ar_hip_tokenizer_encode(const ar_tokenizer* t, const char* text, int64_t text_len, int add_bos,
                                       int add_eos, int32_t* out, int capacity, int* count) {
    if (!t || (!text && text_len) || !count || text_len < 0) {
        ar_set_error("bad argument");
        return AR_HIP_ERR_INVALID;
    }
    std::vector<uint32_t> cps;
    std::vector<size_t> offs;
    if (!utf8_decode(text, (size_t)text_len, &cps, &offs)) {
        ar_set_error("text is not valid UTF-8");
        return AR_HIP_ERR_INVALID;
    }
    std::vector<std::pair<size_t, size_t>> segs;
    pretokenize(cps, &segs);
    const bool special = add_bos || add_eos;  // the base encode adds both, then Qwen3Tokenizer trims
    std::vector<int32_t> ids;
    if (special) ids.push_back(AR_QWEN3_BOS_TOKEN);
    const ByteMap& bm = byte_map();
    std::vector<std::string> toks;
    for (const auto& s : segs) {
        toks.clear();
        for (size_t b = offs[s.first]; b < offs[s.second]; b++) {
            std::string ch;
            put_utf8(ch, bm.to_cp[(unsigned char)text[b]]);
            toks.push_back(std::move(ch));
        }
        for (const std::string& tk : bpe(t, std::move(toks))) {
            auto it = t->ids.find(tk);
            ids.push_back(it == t->ids.end() ? AR_QWEN3_UNK_TOKEN : it->second);
        }
        toks.clear();
    }
    if (special) {
        ids.push_back(AR_QWEN3_EOS_TOKEN);
        if (!add_bos && !ids.empty() && ids.front() == AR_QWEN3_BOS_TOKEN) ids.erase(ids.begin());
        if (!add_eos && !ids.empty() && ids.back() == AR_QWEN3_EOS_TOKEN) ids.pop_back();
    }
    *count = (int)ids.size();
    if (!out) return AR_HIP_OK;
    if ((int)ids.size() > capacity) {
        ar_set_error("%d token ids for room of %d", (int)ids.size(), capacity);
        return AR_HIP_ERR_INVALID;
    }
    std::copy(ids.begin(), ids.end(), out);
    return AR_HIP_OK;
}

extern "C" int ar_hip_tokenizer_decode(const ar_tokenizer* t, const int32_t* ids, int n, char* out, int64_t capacity,
                                       int64_t* length) {
    if (!t || (!ids && n) || n < 0 || !length) {
        ar_set_error("bad argument");
        return AR_HIP_ERR_INVALID;
    }
    std::string bytes;
    const ByteMap& bm = byte_map();
    for (int k = 0; k < n; k++) {
        const int id = ids[k];
        if (is_special(id) || id < 0 || id >= (int)t->vocab.size()) continue;
        const std::string& s = t->vocab[id];
        std::vector<uint32_t> cps;
        std::vector<size_t> offs;
        utf8_decode(s.data(), s.size(), &cps, &offs);  // vocabulary strings are valid UTF-8
        for (uint32_t cp : cps) {
            if (cp >= 512 || bm.from_cp[cp] < 0) {
                ar_set_error("Invalid byte-level character U+%04X in token %d", cp, id);
                return AR_HIP_ERR_INVALID;
            }
            bytes += (char)bm.from_cp[cp];
        }
    }
    const std::string text = utf8_sanitize((const unsigned char*)bytes.data(), bytes.size());
    *length = (int64_t)text.size();
    if (!out) return AR_HIP_OK;
    if ((int64_t)text.size() > capacity) {
        ar_set_error("%lld bytes for room of %lld", (long long)text.size(), (long long)capacity);
        return AR_HIP_ERR_INVALID;
    }
    std::memcpy(out, text.data(), text.size());
    if ((int64_t)text.size() < capacity) out[text.size()] = '\0';
    return AR_HIP_OK;
}
