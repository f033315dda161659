// UTF-8 helpers shared by the host-side tokenizers (tokenizer.cpp, bpe.cpp).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace utf8 {

inline void put_utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
        s += (char)cp;
    } else if (cp < 0x800) {
        s += (char)(0xC0 | (cp >> 6));
        s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        s += (char)(0xE0 | (cp >> 12));
        s += (char)(0x80 | ((cp >> 6) & 0x3F));
        s += (char)(0x80 | (cp & 0x3F));
    } else {
        s += (char)(0xF0 | (cp >> 18));
        s += (char)(0x80 | ((cp >> 12) & 0x3F));
        s += (char)(0x80 | ((cp >> 6) & 0x3F));
        s += (char)(0x80 | (cp & 0x3F));
    }
}

// Length of the well-formed UTF-8 sequence at p (Unicode Table 3-7), or 0; *valid_prefix gets the
// length of its longest well-formed prefix (the "maximal subpart", at least 1).
inline int utf8_seq(const unsigned char* p, size_t n, uint32_t* cp, int* valid_prefix) {
    const unsigned char b0 = p[0];
    *valid_prefix = 1;
    if (b0 < 0x80) {
        *cp = b0;
        return 1;
    }
    int len;
    unsigned char lo = 0x80, hi = 0xBF;
    uint32_t v;
    if (b0 >= 0xC2 && b0 <= 0xDF) {
        len = 2;
        v = b0 & 0x1F;
    } else if (b0 >= 0xE0 && b0 <= 0xEF) {
        len = 3;
        v = b0 & 0x0F;
        if (b0 == 0xE0) lo = 0xA0;
        if (b0 == 0xED) hi = 0x9F;
    } else if (b0 >= 0xF0 && b0 <= 0xF4) {
        len = 4;
        v = b0 & 0x07;
        if (b0 == 0xF0) lo = 0x90;
        if (b0 == 0xF4) hi = 0x8F;
    } else {
        return 0;
    }
    for (int k = 1; k < len; k++) {
        if ((size_t)k >= n) return 0;
        const unsigned char b = p[k];
        const unsigned char l = k == 1 ? lo : 0x80, h = k == 1 ? hi : 0xBF;
        if (b < l || b > h) return 0;
        v = (v << 6) | (b & 0x3F);
        *valid_prefix = k + 1;
    }
    *cp = v;
    return len;
}

// Java's new String(bytes, UTF_8): malformed input replaced by U+FFFD per maximal subpart.
inline std::string utf8_sanitize(const unsigned char* p, size_t n) {
    std::string out;
    out.reserve(n);
    size_t i = 0;
    while (i < n) {
        uint32_t cp;
        int vp;
        const int len = utf8_seq(p + i, n - i, &cp, &vp);
        if (len) {
            out.append((const char*)p + i, (size_t)len);
            i += (size_t)len;
        } else {
            put_utf8(out, 0xFFFD);
            i += (size_t)vp;
        }
    }
    return out;
}

// Strict decode of input text: code points and the byte offset of each (plus the end).
inline bool utf8_decode(const char* text, size_t n, std::vector<uint32_t>* cps, std::vector<size_t>* offs) {
    const unsigned char* p = (const unsigned char*)text;
    size_t i = 0;
    while (i < n) {
        uint32_t cp;
        int vp;
        const int len = utf8_seq(p + i, n - i, &cp, &vp);
        if (!len) return false;
        cps->push_back(cp);
        offs->push_back(i);
        i += (size_t)len;
    }
    offs->push_back(n);
    return true;
}

}  // namespace utf8
