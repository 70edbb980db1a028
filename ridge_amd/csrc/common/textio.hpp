// textio.hpp -- the build's text inputs, read one way everywhere: flat JSON
// hardware descriptions (the model library), '#'-annotated CSV tables
// (ridge-predict's batch mode) and registered shape lists (ridge-measure).
//
// Every reader returns a Status. A failed Status carries one message of the
// form "<where>: <what>", where <where> is a file name, optionally with a line
// number or a byte offset, so a bad input is reported where it is.
#pragma once

#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <set>
#include <sstream>
#include <string>
#include <vector>

namespace ridgeio {

class Status {
public:
    Status() = default;
    static Status failure(const std::string& where, const std::string& what) {
        Status s;
        s.message_ = where.empty() ? what : where + ": " + what;
        return s;
    }
    bool ok() const { return message_.empty(); }
    const std::string& message() const { return message_; }

private:
    std::string message_;
};

inline Status readWholeFile(const std::string& path, std::string& text) {
    std::ifstream in(path, std::ios::binary);
    if (!in) return Status::failure(path, "cannot read (" + std::string(std::strerror(errno)) + ")");
    std::ostringstream buf;
    buf << in.rdbuf();
    text = buf.str();
    return Status();
}

// ---------------------------------------------------------------- numbers --

// True when `s` (surrounding blanks aside) is a decimal number as JSON writes
// one, with an optional leading '+': [+-]? digits [. digits]? ([eE] [+-]? digits)?.
// strtod alone would also take hexadecimal ("0x1p3"), "inf" and "nan".
inline bool isDecimalNumber(const std::string& s) {
    size_t i = 0, n = s.size();
    while (i < n && std::isspace(static_cast<unsigned char>(s[i]))) ++i;
    while (n > i && std::isspace(static_cast<unsigned char>(s[n - 1]))) --n;
    auto digits = [&]() {
        const size_t from = i;
        while (i < n && std::isdigit(static_cast<unsigned char>(s[i]))) ++i;
        return i > from;
    };
    if (i < n && (s[i] == '-' || s[i] == '+')) ++i;
    if (!digits()) return false;
    if (i < n && s[i] == '.') {
        ++i;
        if (!digits()) return false;
    }
    if (i < n && (s[i] == 'e' || s[i] == 'E')) {
        ++i;
        if (i < n && (s[i] == '-' || s[i] == '+')) ++i;
        if (!digits()) return false;
    }
    return i == n;
}

// The whole of `s` (surrounding blanks aside) as a finite real written in
// decimal notation (isDecimalNumber).
inline bool toReal(const std::string& s, double& v) {
    if (!isDecimalNumber(s)) return false;
    const char* b = s.c_str();
    char* e = nullptr;
    errno = 0;
    const double x = std::strtod(b, &e);
    if (e == b || errno == ERANGE || !std::isfinite(x)) return false;
    while (*e && std::isspace(static_cast<unsigned char>(*e))) ++e;
    if (*e) return false;
    v = x;
    return true;
}

// The whole of `s` as an integer. Written forms of an integral real ("108",
// "1.0e3") are accepted; a fractional value is not.
inline bool toInteger(const std::string& s, long long& v) {
    double x = 0.0;
    if (!toReal(s, x) || x != std::floor(x) || std::fabs(x) > 9.0e15) return false;
    v = static_cast<long long>(x);
    return true;
}

// ------------------------------------------------------------- flat JSON --
//
// Accepted: one object whose values are strings, numbers, true, false or null,
// e.g. {"numSMs": 256, "name": "MI355X"}. Keys are unique. Nested objects and
// arrays are refused (the format is flat by definition). String values are
// stored unescaped; every other value is stored as written. `quoted` names the
// keys whose value was a string, so that a numeric field can refuse "256".

struct FlatObject : std::map<std::string, std::string> {
    std::set<std::string> quoted;
};

namespace detail {

struct Token {
    enum Kind { Open, Close, Colon, Comma, Text, Scalar, End, Invalid } kind;
    std::string value;
    size_t offset;
};

class JsonScanner {
public:
    explicit JsonScanner(const std::string& text) : text_(text) {}

    Token next() {
        while (pos_ < text_.size() && std::isspace(static_cast<unsigned char>(text_[pos_]))) ++pos_;
        const size_t at = pos_;
        if (pos_ == text_.size()) return {Token::End, "", at};
        const char c = text_[pos_];
        switch (c) {
            case '{': ++pos_; return {Token::Open, "{", at};
            case '}': ++pos_; return {Token::Close, "}", at};
            case ':': ++pos_; return {Token::Colon, ":", at};
            case ',': ++pos_; return {Token::Comma, ",", at};
            case '"': return quoted(at);
            case '[': return {Token::Invalid, "arrays are not part of the flat format", at};
            default: break;
        }
        size_t end = pos_;
        while (end < text_.size() && (std::isalnum(static_cast<unsigned char>(text_[end])) || text_[end] == '.' ||
                                      text_[end] == '-' || text_[end] == '+'))
            ++end;
        if (end == pos_) return {Token::Invalid, std::string("unexpected character '") + c + "'", at};
        Token t{Token::Scalar, text_.substr(pos_, end - pos_), at};
        pos_ = end;
        double unused = 0.0;
        if (t.value != "true" && t.value != "false" && t.value != "null" && !toReal(t.value, unused))
            return {Token::Invalid, "\"" + t.value + "\" is neither a number nor true, false or null", at};
        return t;
    }

private:
    Token quoted(size_t at) {
        std::string out;
        for (size_t i = at + 1; i < text_.size(); ++i) {
            const char c = text_[i];
            if (c == '"') {
                pos_ = i + 1;
                return {Token::Text, out, at};
            }
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (++i == text_.size()) break;
            static const char kFrom[] = "\"\\/bfnrt";
            static const char kTo[] = "\"\\/\b\f\n\r\t";
            const char* hit = std::strchr(kFrom, text_[i]);
            if (hit && *hit) {
                out.push_back(kTo[hit - kFrom]);
            } else if (text_[i] == 'u' && i + 4 < text_.size()) {
                const unsigned long cp = std::strtoul(text_.substr(i + 1, 4).c_str(), nullptr, 16);
                out.push_back(cp < 0x80 ? static_cast<char>(cp) : '?');
                i += 4;
            } else {
                return {Token::Invalid, "unknown escape in a string", i};
            }
        }
        return {Token::Invalid, "string is not closed", at};
    }

    const std::string& text_;
    size_t pos_ = 0;
};

}  // namespace detail

// Parses `text` (read from `source`, used in messages) into `out`.
inline Status parseFlatObject(const std::string& text, const std::string& source, FlatObject& out) {
    using detail::Token;
    enum class Want { Open, KeyOrClose, Key, Colon, Value, CommaOrClose, Nothing };
    detail::JsonScanner scan(text);
    FlatObject kv;
    std::string key;
    Want want = Want::Open;
    auto fail = [&](const Token& t, const std::string& what) {
        return Status::failure(source + " at byte " + std::to_string(t.offset), what);
    };
    for (;;) {
        const Token t = scan.next();
        if (t.kind == Token::Invalid) return fail(t, t.value);
        if (t.kind == Token::End && want != Want::Nothing)
            return fail(t, want == Want::Open ? "a hardware description is one JSON object" : "the object is not closed");
        switch (want) {
            case Want::Open:
                if (t.kind != Token::Open) return fail(t, "a hardware description is one JSON object");
                want = Want::KeyOrClose;
                break;
            case Want::KeyOrClose:
            case Want::Key:
                if (want == Want::KeyOrClose && t.kind == Token::Close) {
                    want = Want::Nothing;
                    break;
                }
                if (t.kind != Token::Text) return fail(t, "a key (a quoted string) belongs here");
                if (kv.count(t.value)) return fail(t, "key \"" + t.value + "\" appears twice");
                key = t.value;
                want = Want::Colon;
                break;
            case Want::Colon:
                if (t.kind != Token::Colon) return fail(t, "':' belongs after key \"" + key + "\"");
                want = Want::Value;
                break;
            case Want::Value:
                if (t.kind == Token::Open) return fail(t, "nested objects are not part of the flat format");
                if (t.kind != Token::Text && t.kind != Token::Scalar)
                    return fail(t, "key \"" + key + "\" has no value");
                kv[key] = t.value;
                if (t.kind == Token::Text) kv.quoted.insert(key);
                want = Want::CommaOrClose;
                break;
            case Want::CommaOrClose:
                if (t.kind == Token::Comma) {
                    want = Want::Key;
                } else if (t.kind == Token::Close) {
                    want = Want::Nothing;
                } else {
                    return fail(t, "the object continues with ',' or ends with '}'");
                }
                break;
            case Want::Nothing:
                if (t.kind != Token::End) return fail(t, "text after the end of the object");
                out = std::move(kv);
                return Status();
        }
    }
}

// ------------------------------------------------------------ CSV tables --
//
// A '#' line is a comment; blank lines are dropped; the first other line is
// the header and every later one a record. Fields are split on commas (the
// build's tables quote nothing).

inline std::vector<std::string> splitFields(const std::string& line) {
    std::vector<std::string> fields;
    size_t from = 0;
    for (;;) {
        const size_t comma = line.find(',', from);
        fields.push_back(line.substr(from, comma == std::string::npos ? std::string::npos : comma - from));
        if (comma == std::string::npos) return fields;
        from = comma + 1;
    }
}

struct TableLine {
    enum Kind { Comment, Header, Record } kind;
    size_t number;                    // 1-based line number in the file
    std::string text;                 // as written, without the line break
    std::vector<std::string> fields;  // empty for comments
};

inline Status readTable(const std::string& path, std::vector<TableLine>& out) {
    std::string text;
    Status st = readWholeFile(path, text);
    if (!st.ok()) return st;
    std::vector<TableLine> lines;
    bool haveHeader = false;
    size_t number = 0, start = 0;
    while (start < text.size()) {
        size_t stop = text.find('\n', start);
        if (stop == std::string::npos) stop = text.size();
        std::string line = text.substr(start, stop - start);
        start = stop + 1;
        ++number;
        if (!line.empty() && line.back() == '\r') line.pop_back();
        if (line.empty()) continue;
        if (line[0] == '#') {
            lines.push_back({TableLine::Comment, number, line, {}});
            continue;
        }
        lines.push_back({haveHeader ? TableLine::Record : TableLine::Header, number, line, splitFields(line)});
        haveHeader = true;
    }
    if (!haveHeader) return Status::failure(path, "no header line");
    out.swap(lines);
    return Status();
}

// Column name -> position in a header; -1 when absent.
class ColumnIndex {
public:
    explicit ColumnIndex(const std::vector<std::string>& header) {
        for (size_t i = 0; i < header.size(); ++i) pos_.emplace(header[i], static_cast<int>(i));
    }
    int operator[](const std::string& name) const {
        const auto it = pos_.find(name);
        return it == pos_.end() ? -1 : it->second;
    }

private:
    std::map<std::string, int> pos_;
};

// ------------------------------------------------- registered shape lists --
//
// `M,N,K,tag,rationale` records (the header is a comment, as in the
// reference's data/sweep/phase4-registered.csv); only M, N, K and tag are read.

struct Shape {
    long long M = 0, N = 0, K = 0;
    std::string tag;
};

inline Status readShapes(const std::string& path, std::vector<Shape>& out) {
    std::string text;
    Status st = readWholeFile(path, text);
    if (!st.ok()) return st;
    std::vector<Shape> shapes;
    std::istringstream in(text);
    std::string line;
    for (size_t number = 1; std::getline(in, line); ++number) {
        if (!line.empty() && line.back() == '\r') line.pop_back();
        if (line.empty() || line[0] == '#') continue;
        const std::vector<std::string> f = splitFields(line);
        Shape s;
        if (f.size() < 4 || !toInteger(f[0], s.M) || !toInteger(f[1], s.N) || !toInteger(f[2], s.K) || s.M <= 0 ||
            s.N <= 0 || s.K <= 0)
            return Status::failure(path + ":" + std::to_string(number),
                                   "a registered shape is M,N,K,tag[,rationale] with positive M, N and K");
        s.tag = f[3];
        shapes.push_back(s);
    }
    if (shapes.empty()) return Status::failure(path, "registers no shape");
    out.swap(shapes);
    return Status();
}

}  // namespace ridgeio
