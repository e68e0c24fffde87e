// bfi_grammar.hpp — the reference's grammar-string parsers (sample.rs:207-234), host side,
// shared by the allow-mask producer (smp_mask.hip) and bfi_parse_id_union (bfi_host.cpp).
//
// strip_root trims with Rust's str::trim, which strips Unicode White_Space
// (char::is_whitespace) from both ends; strings are UTF-8, as a Rust String is.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace bfig {

// Unicode White_Space (Rust's char::is_whitespace), which str::trim strips.
inline bool rust_ws(uint32_t cp) {
    return (cp >= 0x09 && cp <= 0x0D) || cp == 0x20 || cp == 0x85 || cp == 0xA0 || cp == 0x1680 ||
           (cp >= 0x2000 && cp <= 0x200A) || cp == 0x2028 || cp == 0x2029 || cp == 0x202F || cp == 0x205F ||
           cp == 0x3000;
}
// Code point starting at s[i] and its length in bytes (valid UTF-8 assumed; a lead byte
// whose sequence runs past the end counts as one byte).
inline uint32_t cp_at(const std::string& s, size_t i, size_t* len) {
    const uint8_t c = (uint8_t)s[i];
    int n = c < 0x80 ? 1 : c < 0xE0 ? 2 : c < 0xF0 ? 3 : 4;
    if (i + n > s.size()) n = 1;
    uint32_t cp = n == 1 ? c : n == 2 ? (c & 0x1Fu) : n == 3 ? (c & 0x0Fu) : (c & 0x07u);
    for (int k = 1; k < n; k++) cp = (cp << 6) | ((uint8_t)s[i + k] & 0x3Fu);
    *len = (size_t)n;
    return cp;
}
// str::trim
inline std::string trim(const std::string& s) {
    size_t a = 0, b = s.size(), n;
    while (a < b && rust_ws(cp_at(s, a, &n))) a += n;
    while (b > a) {
        size_t p = b - 1;
        while (p > a && ((uint8_t)s[p] & 0xC0u) == 0x80u) p--;  // start of the last code point
        if (!rust_ws(cp_at(s, p, &n))) break;
        b = p;
    }
    return s.substr(a, b - a);
}
// sample.rs:230-234: trim, "root", trim, "::=", trim; the rest.
inline bool strip_root(const std::string& g, std::string* rest) {
    const std::string s = trim(g);
    if (s.compare(0, 4, "root") != 0) return false;
    const std::string r = trim(s.substr(4));
    if (r.compare(0, 3, "::=") != 0) return false;
    *rest = trim(r.substr(3));
    return true;
}
// str::parse::<u32>: an optional '+', one or more ASCII digits, no overflow.
inline bool parse_u32(const std::string& t0, uint32_t* v) {
    std::string t = t0;
    if (!t.empty() && t[0] == '+') t = t.substr(1);
    if (t.empty()) return false;
    uint64_t x = 0;
    for (char ch : t) {
        if (ch < '0' || ch > '9') return false;
        x = x * 10 + (uint64_t)(ch - '0');
        if (x > 0xFFFFFFFFull) return false;
    }
    *v = (uint32_t)x;
    return true;
}
// sample.rs:207-221: `root ::= id(1) | id(2)` -> the ids (in order, repeats kept).
inline bool parse_id_union(const std::string& g, std::vector<uint32_t>* ids) {
    std::string rest;
    if (!strip_root(g, &rest)) return false;
    size_t p = 0;
    for (;;) {
        const size_t q = rest.find('|', p);
        const std::string part = trim(rest.substr(p, q == std::string::npos ? std::string::npos : q - p));
        if (part.size() < 4 || part.compare(0, 3, "id(") != 0 || part.back() != ')') return false;
        uint32_t v;
        if (!parse_u32(trim(part.substr(3, part.size() - 4)), &v)) return false;
        ids->push_back(v);
        if (q == std::string::npos) break;
        p = q + 1;
    }
    return !ids->empty();
}
// sample.rs:222-228: `root ::= "hello"` -> hello (up to the next quote).
inline bool parse_literal_root(const std::string& g, std::string* lit) {
    std::string rest;
    if (!strip_root(g, &rest) || rest.empty() || rest[0] != '"') return false;
    const size_t end = rest.find('"', 1);
    if (end == std::string::npos) return false;
    *lit = rest.substr(1, end - 1);
    return true;
}

}  // namespace bfig
