// Minimal JSON reader for config.json and manifest.json (the exported-dir
// files model.rs:66-210 and model.rs:742-795 parse with serde_json).
// Values only: no serialisation, no comments, UTF-8 passed through.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "host_common.h"

namespace omg {

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;

    bool is_null() const { return kind == Null; }
    bool has(const std::string& k) const { return kind == Object && obj.count(k) != 0; }
    const Json& operator[](const std::string& k) const {
        static const Json none;
        if (kind != Object) return none;
        auto it = obj.find(k);
        return it == obj.end() ? none : it->second;
    }
    const Json& operator[](size_t i) const {
        static const Json none;
        return (kind == Array && i < arr.size()) ? arr[i] : none;
    }
    // serde_json's as_u64 / as_f64 / as_str / as_bool: absent or wrong kind -> fallback.
    // Whole numbers up to 2^53 (every one exact in a double); anything
    // larger, fractional or non-finite is not an unsigned integer here.
    bool is_uint() const { return kind == Number && num >= 0 && num <= 9007199254740992.0 && double(uint64_t(num)) == num; }
    uint64_t u64(uint64_t fallback) const { return is_uint() ? uint64_t(num) : fallback; }
    double f64(double fallback) const { return kind == Number ? num : fallback; }
    std::string s(const std::string& fallback) const { return kind == String ? str : fallback; }
    bool boolean(bool fallback) const { return kind == Bool ? b : fallback; }

    static Json parse(const std::string& text) {
        size_t i = 0;
        Json v = value(text, i);
        ws(text, i);
        if (i != text.size()) fail(E_INVALID, "json: trailing characters");
        return v;
    }

   private:
    static void ws(const std::string& t, size_t& i) {
        while (i < t.size() && (t[i] == ' ' || t[i] == '\n' || t[i] == '\r' || t[i] == '\t')) ++i;
    }
    static void expect(const std::string& t, size_t& i, const char* lit) {
        for (const char* p = lit; *p; ++p, ++i)
            if (i >= t.size() || t[i] != *p) fail(E_INVALID, std::string("json: expected ") + lit);
    }
    static void put_utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += char(cp);
        } else if (cp < 0x800) {
            out += char(0xc0 | (cp >> 6));
            out += char(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            out += char(0xe0 | (cp >> 12));
            out += char(0x80 | ((cp >> 6) & 0x3f));
            out += char(0x80 | (cp & 0x3f));
        } else {
            out += char(0xf0 | (cp >> 18));
            out += char(0x80 | ((cp >> 12) & 0x3f));
            out += char(0x80 | ((cp >> 6) & 0x3f));
            out += char(0x80 | (cp & 0x3f));
        }
    }
    static std::string string_lit(const std::string& t, size_t& i) {
        std::string out;
        ++i;  // opening quote
        while (true) {
            if (i >= t.size()) fail(E_INVALID, "json: unterminated string");
            char c = t[i++];
            if (c == '"') break;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i >= t.size()) fail(E_INVALID, "json: bad escape");
            char e = t[i++];
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
                    if (i + 4 > t.size()) fail(E_INVALID, "json: bad \\u escape");
                    uint32_t cp = uint32_t(std::strtoul(t.substr(i, 4).c_str(), nullptr, 16));
                    i += 4;
                    if (cp >= 0xd800 && cp < 0xdc00 && i + 6 <= t.size() && t[i] == '\\' && t[i + 1] == 'u') {
                        uint32_t lo = uint32_t(std::strtoul(t.substr(i + 2, 4).c_str(), nullptr, 16));
                        i += 6;
                        cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: fail(E_INVALID, "json: bad escape");
            }
        }
        return out;
    }
    static Json value(const std::string& t, size_t& i) {
        ws(t, i);
        if (i >= t.size()) fail(E_INVALID, "json: unexpected end");
        Json v;
        char c = t[i];
        if (c == '{') {
            v.kind = Object;
            ++i;
            ws(t, i);
            if (i < t.size() && t[i] == '}') {
                ++i;
                return v;
            }
            while (true) {
                ws(t, i);
                if (i >= t.size() || t[i] != '"') fail(E_INVALID, "json: expected key");
                std::string k = string_lit(t, i);
                ws(t, i);
                expect(t, i, ":");
                v.obj[k] = value(t, i);
                ws(t, i);
                if (i < t.size() && t[i] == ',') {
                    ++i;
                    continue;
                }
                expect(t, i, "}");
                break;
            }
        } else if (c == '[') {
            v.kind = Array;
            ++i;
            ws(t, i);
            if (i < t.size() && t[i] == ']') {
                ++i;
                return v;
            }
            while (true) {
                v.arr.push_back(value(t, i));
                ws(t, i);
                if (i < t.size() && t[i] == ',') {
                    ++i;
                    continue;
                }
                expect(t, i, "]");
                break;
            }
        } else if (c == '"') {
            v.kind = String;
            v.str = string_lit(t, i);
        } else if (c == 't') {
            expect(t, i, "true");
            v.kind = Bool;
            v.b = true;
        } else if (c == 'f') {
            expect(t, i, "false");
            v.kind = Bool;
        } else if (c == 'n') {
            expect(t, i, "null");
        } else {
            const char* start = t.c_str() + i;
            char* end = nullptr;
            v.num = std::strtod(start, &end);
            if (end == start) fail(E_INVALID, "json: bad value");
            v.kind = Number;
            i += size_t(end - start);
        }
        return v;
    }
};

}  // namespace omg
