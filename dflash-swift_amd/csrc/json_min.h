/*
 * json_min.h -- a small JSON reader (RFC 8259) for safetensors headers and MLX config.json
 * files.  Values are held in a tree of JsonValue; numbers keep their integer value when the
 * text is an integer that fits int64.  Parse errors carry the byte offset.
 */
#ifndef DFQ_JSON_MIN_H
#define DFQ_JSON_MIN_H

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace dfq {

struct JsonValue {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    bool is_int = false;
    int64_t i = 0;
    std::string str;
    std::vector<JsonValue> arr;
    /* object members in document order (duplicate keys: the last one wins in find) */
    std::vector<std::pair<std::string, JsonValue>> obj;

    const JsonValue* find(const std::string& key) const {
        for (auto it = obj.rbegin(); it != obj.rend(); ++it)
            if (it->first == key) return &it->second;
        return nullptr;
    }
};

class JsonParser {
public:
    JsonParser(const char* s, size_t n) : s_(s), n_(n) {}

    /* Parses one value filling the whole input (whitespace aside).  On failure returns
     * false and sets err to a message with the offset. */
    bool parse(JsonValue* out, std::string* err) {
        pos_ = 0;
        depth_ = 0;
        err_.clear();
        skip_ws();
        if (!value(out)) {
            *err = err_;
            return false;
        }
        skip_ws();
        if (pos_ != n_) {
            *err = "trailing characters at offset " + std::to_string(pos_);
            return false;
        }
        return true;
    }

private:
    const char* s_;
    size_t n_;
    size_t pos_ = 0;
    int depth_ = 0;
    std::string err_;

    bool fail(const char* what) {
        err_ = std::string(what) + " at offset " + std::to_string(pos_);
        return false;
    }
    void skip_ws() {
        while (pos_ < n_ && (s_[pos_] == ' ' || s_[pos_] == '\t' || s_[pos_] == '\n' ||
                             s_[pos_] == '\r'))
            ++pos_;
    }
    bool literal(const char* lit) {
        size_t k = 0;
        while (lit[k]) {
            if (pos_ + k >= n_ || s_[pos_ + k] != lit[k]) return fail("bad literal");
            ++k;
        }
        pos_ += k;
        return true;
    }
    bool value(JsonValue* v) {
        if (pos_ >= n_) return fail("unexpected end");
        if (++depth_ > 64) return fail("nesting too deep");
        bool ok;
        switch (s_[pos_]) {
            case '{': ok = object(v); break;
            case '[': ok = array(v); break;
            case '"': v->kind = JsonValue::String; ok = string(&v->str); break;
            case 't': v->kind = JsonValue::Bool; v->b = true; ok = literal("true"); break;
            case 'f': v->kind = JsonValue::Bool; v->b = false; ok = literal("false"); break;
            case 'n': v->kind = JsonValue::Null; ok = literal("null"); break;
            default: ok = number(v); break;
        }
        --depth_;
        return ok;
    }
    bool object(JsonValue* v) {
        v->kind = JsonValue::Object;
        ++pos_;  // '{'
        skip_ws();
        if (pos_ < n_ && s_[pos_] == '}') {
            ++pos_;
            return true;
        }
        for (;;) {
            skip_ws();
            if (pos_ >= n_ || s_[pos_] != '"') return fail("expected a member name");
            std::string key;
            if (!string(&key)) return false;
            skip_ws();
            if (pos_ >= n_ || s_[pos_] != ':') return fail("expected ':'");
            ++pos_;
            skip_ws();
            v->obj.emplace_back(std::move(key), JsonValue{});
            if (!value(&v->obj.back().second)) return false;
            skip_ws();
            if (pos_ < n_ && s_[pos_] == ',') {
                ++pos_;
                continue;
            }
            if (pos_ < n_ && s_[pos_] == '}') {
                ++pos_;
                return true;
            }
            return fail("expected ',' or '}'");
        }
    }
    bool array(JsonValue* v) {
        v->kind = JsonValue::Array;
        ++pos_;  // '['
        skip_ws();
        if (pos_ < n_ && s_[pos_] == ']') {
            ++pos_;
            return true;
        }
        for (;;) {
            skip_ws();
            v->arr.emplace_back();
            if (!value(&v->arr.back())) return false;
            skip_ws();
            if (pos_ < n_ && s_[pos_] == ',') {
                ++pos_;
                continue;
            }
            if (pos_ < n_ && s_[pos_] == ']') {
                ++pos_;
                return true;
            }
            return fail("expected ',' or ']'");
        }
    }
    static void put_utf8(std::string* o, uint32_t c) {
        if (c < 0x80) {
            o->push_back((char)c);
        } else if (c < 0x800) {
            o->push_back((char)(0xC0 | (c >> 6)));
            o->push_back((char)(0x80 | (c & 0x3F)));
        } else if (c < 0x10000) {
            o->push_back((char)(0xE0 | (c >> 12)));
            o->push_back((char)(0x80 | ((c >> 6) & 0x3F)));
            o->push_back((char)(0x80 | (c & 0x3F)));
        } else {
            o->push_back((char)(0xF0 | (c >> 18)));
            o->push_back((char)(0x80 | ((c >> 12) & 0x3F)));
            o->push_back((char)(0x80 | ((c >> 6) & 0x3F)));
            o->push_back((char)(0x80 | (c & 0x3F)));
        }
    }
    bool hex4(uint32_t* out) {
        if (pos_ + 4 > n_) return fail("short \\u escape");
        uint32_t c = 0;
        for (int k = 0; k < 4; ++k) {
            const char h = s_[pos_ + k];
            c <<= 4;
            if (h >= '0' && h <= '9') c |= (uint32_t)(h - '0');
            else if (h >= 'a' && h <= 'f') c |= (uint32_t)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') c |= (uint32_t)(h - 'A' + 10);
            else return fail("bad hex digit");
        }
        pos_ += 4;
        *out = c;
        return true;
    }
    bool string(std::string* o) {
        ++pos_;  // '"'
        for (;;) {
            if (pos_ >= n_) return fail("unterminated string");
            const unsigned char c = (unsigned char)s_[pos_];
            if (c == '"') {
                ++pos_;
                return true;
            }
            if (c < 0x20) return fail("control character in string");
            if (c != '\\') {
                o->push_back((char)c);
                ++pos_;
                continue;
            }
            if (++pos_ >= n_) return fail("unterminated escape");
            const char e = s_[pos_++];
            switch (e) {
                case '"': o->push_back('"'); break;
                case '\\': o->push_back('\\'); break;
                case '/': o->push_back('/'); break;
                case 'b': o->push_back('\b'); break;
                case 'f': o->push_back('\f'); break;
                case 'n': o->push_back('\n'); break;
                case 'r': o->push_back('\r'); break;
                case 't': o->push_back('\t'); break;
                case 'u': {
                    uint32_t c1 = 0;
                    if (!hex4(&c1)) return false;
                    if (c1 >= 0xD800 && c1 < 0xDC00) {  // a surrogate pair
                        uint32_t c2 = 0;
                        if (pos_ + 2 > n_ || s_[pos_] != '\\' || s_[pos_ + 1] != 'u')
                            return fail("lone high surrogate");
                        pos_ += 2;
                        if (!hex4(&c2)) return false;
                        if (c2 < 0xDC00 || c2 >= 0xE000) return fail("bad low surrogate");
                        c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
                    } else if (c1 >= 0xDC00 && c1 < 0xE000) {
                        return fail("lone low surrogate");
                    }
                    put_utf8(o, c1);
                    break;
                }
                default: return fail("bad escape");
            }
        }
    }
    bool number(JsonValue* v) {
        const size_t start = pos_;
        if (pos_ < n_ && s_[pos_] == '-') ++pos_;
        if (pos_ >= n_ || s_[pos_] < '0' || s_[pos_] > '9') return fail("bad value");
        if (s_[pos_] == '0') {
            ++pos_;
        } else {
            while (pos_ < n_ && s_[pos_] >= '0' && s_[pos_] <= '9') ++pos_;
        }
        bool integral = true;
        if (pos_ < n_ && s_[pos_] == '.') {
            integral = false;
            ++pos_;
            if (pos_ >= n_ || s_[pos_] < '0' || s_[pos_] > '9') return fail("bad fraction");
            while (pos_ < n_ && s_[pos_] >= '0' && s_[pos_] <= '9') ++pos_;
        }
        if (pos_ < n_ && (s_[pos_] == 'e' || s_[pos_] == 'E')) {
            integral = false;
            ++pos_;
            if (pos_ < n_ && (s_[pos_] == '+' || s_[pos_] == '-')) ++pos_;
            if (pos_ >= n_ || s_[pos_] < '0' || s_[pos_] > '9') return fail("bad exponent");
            while (pos_ < n_ && s_[pos_] >= '0' && s_[pos_] <= '9') ++pos_;
        }
        const std::string text(s_ + start, pos_ - start);
        v->kind = JsonValue::Number;
        v->num = std::strtod(text.c_str(), nullptr);
        v->is_int = false;
        if (integral) {
            /* exact int64 when it fits: accumulate with an overflow check */
            const bool neg = text[0] == '-';
            uint64_t acc = 0;
            bool fits = true;
            for (size_t k = neg ? 1 : 0; k < text.size(); ++k) {
                const uint64_t d = (uint64_t)(text[k] - '0');
                if (acc > (UINT64_MAX - d) / 10) {
                    fits = false;
                    break;
                }
                acc = acc * 10 + d;
            }
            const uint64_t lim = neg ? (uint64_t)INT64_MAX + 1 : (uint64_t)INT64_MAX;
            if (fits && acc <= lim) {
                v->is_int = true;
                v->i = neg ? (int64_t)(0 - acc) : (int64_t)acc;
            }
        }
        return true;
    }
};

}  // namespace dfq

#endif
