// Minimal JSON reader (host code) for the headers of model files: objects, arrays,
// strings with escapes, integers, other numbers, true/false/null, with a depth limit.
// Either skips values, reads the few shapes the safetensors header needs, or builds a
// small document tree (the model graph).
#pragma once
#include <stdint.h>

#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace ppocr {

// A parsed JSON value.
struct JVal {
    enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
    bool b = false;
    double num = 0.0;
    bool is_int = false;
    int64_t i = 0;
    std::string s;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal* get(const char* key) const {
        if (kind != kObj) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

struct Json {
    const char* p;
    const char* end;
    std::string err;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool expect(char c) {
        ws();
        if (p >= end || *p != c) {
            err = std::string("expected '") + c + "'";
            return false;
        }
        ++p;
        return true;
    }
    bool peek(char c) {
        ws();
        return p < end && *p == c;
    }
    bool string(std::string* out) {
        if (!expect('"')) return false;
        std::string s;
        while (p < end && *p != '"') {
            char c = *p++;
            if ((unsigned char)c < 0x20) {
                err = "control character in string";
                return false;
            }
            if (c == '\\') {
                if (p >= end) break;
                const char e = *p++;
                switch (e) {
                    case '"': s += '"'; break;
                    case '\\': s += '\\'; break;
                    case '/': s += '/'; break;
                    case 'b': s += '\b'; break;
                    case 'f': s += '\f'; break;
                    case 'n': s += '\n'; break;
                    case 'r': s += '\r'; break;
                    case 't': s += '\t'; break;
                    case 'u': {
                        if (end - p < 4) {
                            err = "truncated \\u escape";
                            return false;
                        }
                        unsigned v = 0;
                        for (int x = 0; x < 4; ++x) {
                            const char h = *p++;
                            v <<= 4;
                            if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
                            else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
                            else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
                            else {
                                err = "bad \\u escape";
                                return false;
                            }
                        }
                        // names are compared byte for byte: keep BMP code points as UTF-8
                        if (v < 0x80) {
                            s += (char)v;
                        } else if (v < 0x800) {
                            s += (char)(0xC0 | (v >> 6));
                            s += (char)(0x80 | (v & 0x3F));
                        } else {
                            s += (char)(0xE0 | (v >> 12));
                            s += (char)(0x80 | ((v >> 6) & 0x3F));
                            s += (char)(0x80 | (v & 0x3F));
                        }
                        break;
                    }
                    default: err = "bad escape"; return false;
                }
            } else {
                s += c;
            }
        }
        if (p >= end) {
            err = "unterminated string";
            return false;
        }
        ++p;  // closing quote
        if (out) *out = std::move(s);
        return true;
    }
    bool integer(int64_t* out) {
        ws();
        const char* q = p;
        if (q < end && *q == '-') ++q;
        if (q >= end || *q < '0' || *q > '9') {
            err = "expected an integer";
            return false;
        }
        bool neg = *p == '-';
        if (neg) ++p;
        uint64_t v = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            const uint64_t d = (uint64_t)(*p - '0');
            if (v > (UINT64_MAX - d) / 10) {
                err = "integer overflow";
                return false;
            }
            v = v * 10 + d;
            ++p;
        }
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) {
            err = "expected an integer";
            return false;
        }
        if (v > (uint64_t)INT64_MAX) {
            err = "integer overflow";
            return false;
        }
        *out = neg ? -(int64_t)v : (int64_t)v;
        return true;
    }
    // Skips any value (depth-limited).
    bool skip(int depth = 0) {
        if (depth > 64) {
            err = "nesting too deep";
            return false;
        }
        ws();
        if (p >= end) {
            err = "unexpected end";
            return false;
        }
        if (*p == '"') return string(nullptr);
        if (*p == '{') {
            ++p;
            if (peek('}')) return ++p, true;
            do {
                if (!string(nullptr) || !expect(':') || !skip(depth + 1)) return false;
            } while (peek(',') && ++p);
            return expect('}');
        }
        if (*p == '[') {
            ++p;
            if (peek(']')) return ++p, true;
            do {
                if (!skip(depth + 1)) return false;
            } while (peek(',') && ++p);
            return expect(']');
        }
        for (const char* lit : {"true", "false", "null"}) {
            const size_t l = std::strlen(lit);
            if ((size_t)(end - p) >= l && std::memcmp(p, lit, l) == 0) {
                p += l;
                return true;
            }
        }
        // a number (any form)
        const char* q = p;
        while (p < end && (std::strchr("+-.eE", *p) || (*p >= '0' && *p <= '9'))) ++p;
        if (p == q) {
            err = "unexpected character";
            return false;
        }
        return true;
    }
    bool int_array(std::vector<int64_t>* out) {
        if (!expect('[')) return false;
        out->clear();
        if (peek(']')) return ++p, true;
        do {
            int64_t v;
            if (!integer(&v)) return false;
            out->push_back(v);
        } while (peek(',') && ++p);
        return expect(']');
    }
    // Parses one value into a tree (depth-limited).
    bool value(JVal* out, int depth = 0) {
        if (depth > 64) {
            err = "nesting too deep";
            return false;
        }
        ws();
        if (p >= end) {
            err = "unexpected end";
            return false;
        }
        if (*p == '"') {
            out->kind = JVal::kStr;
            return string(&out->s);
        }
        if (*p == '{') {
            ++p;
            out->kind = JVal::kObj;
            if (peek('}')) return ++p, true;
            do {
                std::pair<std::string, JVal> kv;
                if (!string(&kv.first) || !expect(':') || !value(&kv.second, depth + 1)) return false;
                out->obj.push_back(std::move(kv));
            } while (peek(',') && ++p);
            return expect('}');
        }
        if (*p == '[') {
            ++p;
            out->kind = JVal::kArr;
            if (peek(']')) return ++p, true;
            do {
                out->arr.emplace_back();
                if (!value(&out->arr.back(), depth + 1)) return false;
            } while (peek(',') && ++p);
            return expect(']');
        }
        if ((size_t)(end - p) >= 4 && std::memcmp(p, "true", 4) == 0) {
            p += 4;
            out->kind = JVal::kBool;
            out->b = true;
            return true;
        }
        if ((size_t)(end - p) >= 5 && std::memcmp(p, "false", 5) == 0) {
            p += 5;
            out->kind = JVal::kBool;
            return true;
        }
        if ((size_t)(end - p) >= 4 && std::memcmp(p, "null", 4) == 0) {
            p += 4;
            return true;
        }
        const char* q = p;
        while (p < end && (std::strchr("+-.eE", *p) || (*p >= '0' && *p <= '9'))) ++p;
        if (p == q) {
            err = "unexpected character";
            return false;
        }
        const std::string t(q, p);
        out->kind = JVal::kNum;
        char* e = nullptr;
        out->num = std::strtod(t.c_str(), &e);
        if (!e || *e) {
            err = "bad number";
            return false;
        }
        if (t.find_first_of(".eE") == std::string::npos) {
            errno = 0;
            const long long v = std::strtoll(t.c_str(), &e, 10);
            if (errno == 0 && e && !*e) {
                out->is_int = true;
                out->i = v;
            }
        }
        return true;
    }
};


}  // namespace ppocr
