// Weight ingestion (include/mamba3_checkpoint.h): the reference's JSON
// checkpoints (src/train/checkpoint.rs:16-83) and state dicts
// (src/nn/module.rs:297-345), read and written on the host.
//
// Reading is two passes over a memory-mapped file.  The first walks the JSON
// structure on one thread, collecting names and shapes and recording where
// each `data` array lies without parsing its numbers (a number never contains
// ']', so the array's end is a byte search).  The second splits the arrays
// into pieces of about kPiece bytes at commas and parses the pieces on
// several threads, each into its own buffer, which are then joined in order.
// A checkpoint of config 4's model is about 163 M values (1.6 GB of text).
#include "mamba3_checkpoint.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace m3 {
m3_status api_fail(m3_status st, const char *fmt, ...);
m3_status api_ok();
}  // namespace m3

struct m3_state_dict {
    struct Entry {
        std::string name;
        std::vector<size_t> shape;
        std::vector<float> data;
    };
    std::vector<Entry> entries;   // key order
    uint64_t step = 0;
    std::string metadata = "null";
};

namespace {

constexpr size_t kPiece = size_t(4) << 20;

int worker_count() {
    unsigned hw = std::thread::hardware_concurrency();
    if (hw == 0) hw = 1;
    if (const char *v = std::getenv("OMP_NUM_THREADS")) {
        const int n = std::atoi(v);
        if (n > 0) hw = std::min<unsigned>(hw, static_cast<unsigned>(n));
    }
    return static_cast<int>(std::min<unsigned>(hw, 16));
}

// Runs f(i) for i in [0, n) on up to worker_count() threads.
template <typename F> void parallel_for(size_t n, F f) {
    const int w = static_cast<int>(std::min<size_t>(n, static_cast<size_t>(worker_count())));
    if (w <= 1) {
        for (size_t i = 0; i < n; ++i) f(i);
        return;
    }
    std::atomic<size_t> next{0};
    std::vector<std::thread> pool;
    for (int t = 0; t < w; ++t)
        pool.emplace_back([&]() {
            for (size_t i = next.fetch_add(1); i < n; i = next.fetch_add(1)) f(i);
        });
    for (auto &th : pool) th.join();
}

// ---------------------------------------------------------------- mapped file
struct Mapped {
    const char *p = nullptr;
    size_t n = 0;
    int fd = -1;
    ~Mapped() {
        if (p && n) munmap(const_cast<char *>(p), n);
        if (fd >= 0) close(fd);
    }
};

m3_status map_file(const char *path, Mapped &m) {
    m.fd = open(path, O_RDONLY);
    if (m.fd < 0) return m3::api_fail(M3_ERR_IO, "%s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(m.fd, &st) != 0) return m3::api_fail(M3_ERR_IO, "%s: %s", path, strerror(errno));
    m.n = static_cast<size_t>(st.st_size);
    if (m.n == 0) return m3::api_ok();
    void *p = mmap(nullptr, m.n, PROT_READ, MAP_PRIVATE, m.fd, 0);
    if (p == MAP_FAILED) {
        m.n = 0;
        return m3::api_fail(M3_ERR_IO, "%s: %s", path, strerror(errno));
    }
    madvise(p, m.n, MADV_SEQUENTIAL);
    m.p = static_cast<const char *>(p);
    return m3::api_ok();
}

// ---------------------------------------------------------------- structure pass
struct Span {
    size_t entry;
    const char *b, *e;   // the array's contents, between '[' and ']'
};

class Parser {
public:
    Parser(const char *b, size_t n) : base_(b), p_(b), end_(b + n) {}

    bool failed() const { return !msg_.empty(); }
    m3_status report() const {
        // line / column as serde_json reports them (1-based line, column of the byte)
        size_t line = 1, col = 0;
        for (const char *q = base_; q < err_at_ && q < end_; ++q) {
            if (*q == '\n') {
                ++line;
                col = 0;
            } else {
                ++col;
            }
        }
        return m3::api_fail(M3_ERR_JSON, "%s at line %zu column %zu", msg_.c_str(), line, col);
    }

    bool parse_file(bool checkpoint, m3_state_dict &sd, std::vector<Span> &spans) {
        ws();
        if (!take('{')) return fail_here(p_ >= end_ ? "EOF while parsing a value" : "expected `{`");
        bool seen_step = false, seen_state = false, seen_entries = false;
        ws();
        if (peek() != '}') {
            for (;;) {
                std::string key;
                ws();
                if (!string(key)) return false;
                ws();
                if (!take(':')) return fail_here("expected `:`");
                ws();
                if (checkpoint && key == "step") {
                    if (!u64(sd.step)) return false;
                    seen_step = true;
                } else if (checkpoint && key == "state") {
                    if (!state_dict_object(sd, spans, seen_entries)) return false;
                    seen_state = true;
                } else if (checkpoint && key == "metadata") {
                    const char *b = p_;
                    if (!skip_value()) return false;
                    sd.metadata.assign(b, p_);
                } else if (!checkpoint && key == "entries") {
                    if (!entries_object(sd, spans)) return false;
                    seen_entries = true;
                } else if (!skip_value()) {
                    return false;
                }
                ws();
                if (take(',')) continue;
                if (take('}')) break;
                return fail_sep(true);
            }
        } else {
            ++p_;
        }
        ws();
        if (p_ != end_) return fail_here("trailing characters");
        if (checkpoint && !seen_step) return fail_here("missing field `step`");
        if (checkpoint && !seen_state) return fail_here("missing field `state`");
        if (!checkpoint && !seen_entries) return fail_here("missing field `entries`");
        return true;
    }

    // Validates one JSON value (used for metadata handed to the writer).
    bool whole_value() {
        ws();
        if (!skip_value()) return false;
        ws();
        return p_ == end_ || fail_here("trailing characters");
    }

private:
    const char *base_, *p_, *end_;
    const char *err_at_ = nullptr;
    std::string msg_;

    bool fail_here(const char *m) {
        if (msg_.empty()) {
            msg_ = m;
            err_at_ = p_;
        }
        return false;
    }
    // a missing separator, or the end of the input where one was due
    bool fail_sep(bool object) {
        if (p_ >= end_) return fail_here(object ? "EOF while parsing an object" : "EOF while parsing a list");
        return fail_here(object ? "expected `,` or `}`" : "expected `,` or `]`");
    }
    char peek() const { return p_ < end_ ? *p_ : '\0'; }
    bool take(char c) {
        if (p_ < end_ && *p_ == c) {
            ++p_;
            return true;
        }
        return false;
    }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\t' || *p_ == '\r')) ++p_;
    }

    static void put_utf8(std::string &o, uint32_t cp) {
        if (cp < 0x80) {
            o += static_cast<char>(cp);
        } else if (cp < 0x800) {
            o += static_cast<char>(0xC0 | (cp >> 6));
            o += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            o += static_cast<char>(0xE0 | (cp >> 12));
            o += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            o += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            o += static_cast<char>(0xF0 | (cp >> 18));
            o += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            o += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            o += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t &v) {
        if (end_ - p_ < 4) return fail_here("EOF while parsing a string");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
            else return fail_here("invalid escape");
        }
        return true;
    }
    // A JSON string at p_ (the opening quote included); `out` gets its value.
    bool string(std::string &out) {
        if (!take('"')) return fail_here("expected `\"`");
        out.clear();
        for (;;) {
            if (p_ >= end_) return fail_here("EOF while parsing a string");
            const char c = *p_++;
            if (c == '"') return true;
            if (static_cast<unsigned char>(c) < 0x20)
                return fail_here("control character (\\u0000-\\u001F) found while parsing a string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ >= end_) return fail_here("EOF while parsing a string");
            const char e = *p_++;
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
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        uint32_t lo;
                        if (!(take('\\') && take('u'))) return fail_here("lone leading surrogate in hex escape");
                        if (!hex4(lo)) return false;
                        if (lo < 0xDC00 || lo >= 0xE000) return fail_here("lone leading surrogate in hex escape");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail_here("lone leading surrogate in hex escape");
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return fail_here("invalid escape");
            }
        }
    }
    bool u64(uint64_t &v) {
        const char *b = p_;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ == b) return fail_here("invalid type: expected an unsigned integer");
        if (p_ < end_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E'))
            return fail_here("invalid type: floating point, expected an unsigned integer");
        const auto r = std::from_chars(b, p_, v);
        if (r.ec != std::errc()) return fail_here("number out of range");
        return true;
    }
    bool literal(const char *w) {
        const size_t n = strlen(w);
        if (static_cast<size_t>(end_ - p_) < n || memcmp(p_, w, n) != 0) return fail_here("expected value");
        p_ += n;
        return true;
    }
    bool number() {
        const char *b = p_;
        take('-');
        if (!(p_ < end_ && *p_ >= '0' && *p_ <= '9')) return fail_here("invalid number");
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                             *p_ == '+' || *p_ == '-'))
            ++p_;
        double d;
        if (std::from_chars(b, p_, d).ec == std::errc::invalid_argument) return fail_here("invalid number");
        return true;
    }
    bool skip_value(int depth = 0) {
        if (depth > 128) return fail_here("recursion limit exceeded");
        ws();
        const char c = peek();
        if (c == '"') {
            std::string s;
            return string(s);
        }
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            ++p_;
            ws();
            if (take(close)) return true;
            for (;;) {
                ws();
                if (c == '{') {
                    std::string k;
                    if (!string(k)) return false;
                    ws();
                    if (!take(':')) return fail_here("expected `:`");
                }
                if (!skip_value(depth + 1)) return false;
                ws();
                if (take(',')) continue;
                if (take(close)) return true;
                return fail_sep(c == '{');
            }
        }
        if (c == 't') return literal("true");
        if (c == 'f') return literal("false");
        if (c == 'n') return literal("null");
        if (c == '-' || (c >= '0' && c <= '9')) return number();
        return fail_here(p_ >= end_ ? "EOF while parsing a value" : "expected value");
    }
    bool state_dict_object(m3_state_dict &sd, std::vector<Span> &spans, bool &seen) {
        if (!take('{')) return fail_here("invalid type: expected struct StateDict");
        ws();
        if (take('}')) return fail_here("missing field `entries`");
        for (;;) {
            std::string key;
            ws();
            if (!string(key)) return false;
            ws();
            if (!take(':')) return fail_here("expected `:`");
            ws();
            if (key == "entries") {
                if (!entries_object(sd, spans)) return false;
                seen = true;
            } else if (!skip_value()) {
                return false;
            }
            ws();
            if (take(',')) continue;
            if (take('}')) break;
            return fail_sep(true);
        }
        return seen || fail_here("missing field `entries`");
    }
    bool entries_object(m3_state_dict &sd, std::vector<Span> &spans) {
        if (!take('{')) return fail_here("invalid type: expected a map");
        ws();
        if (take('}')) return true;
        for (;;) {
            std::string name;
            ws();
            if (!string(name)) return false;
            ws();
            if (!take(':')) return fail_here("expected `:`");
            ws();
            m3_state_dict::Entry e;
            e.name = std::move(name);
            const char *db = nullptr, *de = nullptr;
            if (!tensor_data(e, db, de)) return false;
            // BTreeMap insertion: a repeated key replaces the earlier value
            size_t idx = sd.entries.size();
            for (size_t i = 0; i < sd.entries.size(); ++i)
                if (sd.entries[i].name == e.name) idx = i;
            if (idx == sd.entries.size()) {
                sd.entries.push_back(std::move(e));
            } else {
                sd.entries[idx] = std::move(e);
                spans.erase(std::remove_if(spans.begin(), spans.end(),
                                           [&](const Span &s) { return s.entry == idx; }),
                            spans.end());
            }
            spans.push_back(Span{idx, db, de});
            ws();
            if (take(',')) continue;
            if (take('}')) return true;
            return fail_sep(true);
        }
    }
    bool tensor_data(m3_state_dict::Entry &e, const char *&db, const char *&de) {
        if (!take('{')) return fail_here("invalid type: expected struct TensorData");
        bool shape = false, data = false;
        ws();
        if (!take('}')) {
            for (;;) {
                std::string key;
                ws();
                if (!string(key)) return false;
                ws();
                if (!take(':')) return fail_here("expected `:`");
                ws();
                if (key == "shape") {
                    if (!take('[')) return fail_here("invalid type: expected a sequence");
                    e.shape.clear();
                    ws();
                    if (!take(']')) {
                        for (;;) {
                            uint64_t d;
                            ws();
                            if (!u64(d)) return false;
                            e.shape.push_back(static_cast<size_t>(d));
                            ws();
                            if (take(',')) continue;
                            if (take(']')) break;
                            return fail_sep(false);
                        }
                    }
                    shape = true;
                } else if (key == "data") {
                    if (!take('[')) return fail_here("invalid type: expected a sequence");
                    const void *close = memchr(p_, ']', static_cast<size_t>(end_ - p_));
                    if (close == nullptr) {
                        p_ = end_;
                        return fail_here("EOF while parsing a list");
                    }
                    db = p_;
                    de = static_cast<const char *>(close);
                    p_ = de + 1;
                    data = true;
                } else if (!skip_value()) {
                    return false;
                }
                ws();
                if (take(',')) continue;
                if (take('}')) break;
                return fail_sep(true);
            }
        }
        if (!shape) return fail_here("missing field `shape`");
        if (!data) return fail_here("missing field `data`");
        return true;
    }
};

// ---------------------------------------------------------------- number pass
struct Piece {
    size_t span;
    const char *b, *e;   // values separated by commas; no comma at either end
    bool sole;           // the array's only piece (which may hold no value: `[ ]`)
    std::vector<float> out;
    const char *err = nullptr;   // first bad byte
    const char *why = nullptr;
};

inline bool is_ws(char c) { return c == ' ' || c == '\n' || c == '\t' || c == '\r'; }

// One JSON number as f32: integers go straight to f32 (serde's visit_i64 /
// visit_u64 followed by `as f32`), others through the nearest double.
inline bool parse_f32(const char *b, const char *e, float &v) {
    bool integral = true;
    for (const char *q = b; q < e; ++q)
        if (*q == '.' || *q == 'e' || *q == 'E') {
            integral = false;
            break;
        }
    if (integral) {
        if (*b == '-') {
            int64_t i;
            const auto r = std::from_chars(b, e, i);
            if (r.ec == std::errc() && r.ptr == e) {
                v = i == 0 ? -0.0f : static_cast<float>(i);   // serde_json reads `-0` as -0.0
                return true;
            }
        } else {
            uint64_t u;
            const auto r = std::from_chars(b, e, u);
            if (r.ec == std::errc() && r.ptr == e) {
                v = static_cast<float>(u);
                return true;
            }
        }
    }
    double d;
    const auto r = std::from_chars(b, e, d);
    if (r.ptr != e) return false;
    if (r.ec == std::errc::result_out_of_range) {
        // serde_json: overflow is an error, underflow rounds to zero
        bool neg_exp = false;
        for (const char *q = b; q < e; ++q)
            if ((*q == 'e' || *q == 'E') && q + 1 < e && q[1] == '-') neg_exp = true;
        if (!neg_exp) return false;
        d = (*b == '-') ? -0.0 : 0.0;
    } else if (r.ec != std::errc()) {
        return false;
    }
    v = static_cast<float>(d);
    return true;
}

void parse_piece(Piece &pc) {
    const char *p = pc.b, *e = pc.e;
    pc.out.reserve(static_cast<size_t>(e - p) / 8 + 1);
    while (p < e) {
        while (p < e && is_ws(*p)) ++p;
        if (p >= e) break;
        const char *tb = p;
        if (*p == 'n') {
            pc.err = p;
            pc.why = "invalid type: null, expected f32";
            return;
        }
        if (!(*p == '-' || (*p >= '0' && *p <= '9'))) {
            pc.err = p;
            pc.why = "expected value";
            return;
        }
        while (p < e && *p != ',' && !is_ws(*p)) ++p;
        float v;
        if (!parse_f32(tb, p, v)) {
            pc.err = tb;
            pc.why = "invalid number";
            return;
        }
        pc.out.push_back(v);
        while (p < e && is_ws(*p)) ++p;
        if (p < e) {
            if (*p != ',') {
                pc.err = p;
                pc.why = "expected `,` or `]`";
                return;
            }
            ++p;
            // a comma must be followed by a value
            const char *q = p;
            while (q < e && is_ws(*q)) ++q;
            if (q >= e) {
                pc.err = q;
                pc.why = "trailing comma";
                return;
            }
        }
    }
    if (pc.out.empty() && !pc.sole) {
        pc.err = p;
        pc.why = "expected value";
    }
}

m3_status load(const char *path, bool checkpoint, m3_state_dict **out) {
    if (path == nullptr || out == nullptr) return m3::api_fail(M3_ERR_ARGUMENT, "path or output is NULL");
    *out = nullptr;
    Mapped m;
    m3_status st = map_file(path, m);
    if (st != M3_OK) return st;
    auto *sd = new m3_state_dict();
    std::vector<Span> spans;
    Parser ps(m.p, m.n);
    if (!ps.parse_file(checkpoint, *sd, spans)) {
        delete sd;
        return ps.report();
    }
    // split every data array into pieces at commas
    std::vector<Piece> pieces;
    for (size_t s = 0; s < spans.size(); ++s) {
        const char *b = spans[s].b, *e = spans[s].e;
        const size_t first = pieces.size();
        while (b < e) {
            // cut at a comma; the comma separates this piece from the next
            const char *cut = e, *next = e;
            if (static_cast<size_t>(e - b) > kPiece) {
                const void *c = memchr(b + kPiece, ',', static_cast<size_t>(e - (b + kPiece)));
                if (c != nullptr) {
                    cut = static_cast<const char *>(c);
                    next = cut + 1;
                }
            }
            Piece pc;
            pc.span = s;
            pc.b = b;
            pc.e = cut;
            pc.sole = false;
            pieces.push_back(std::move(pc));
            b = next;
            if (b == e && cut != e) {      // a comma right before ']'
                Piece tail;
                tail.span = s;
                tail.b = tail.e = e;
                tail.sole = false;
                pieces.push_back(std::move(tail));
            }
        }
        if (pieces.size() == first + 1) pieces.back().sole = true;
    }
    parallel_for(pieces.size(), [&](size_t i) { parse_piece(pieces[i]); });
    for (const Piece &pc : pieces) {
        if (pc.err != nullptr) {
            size_t line = 1, col = 0;
            for (const char *q = m.p; q < pc.err; ++q) {
                if (*q == '\n') {
                    ++line;
                    col = 0;
                } else {
                    ++col;
                }
            }
            delete sd;
            return m3::api_fail(M3_ERR_JSON, "%s at line %zu column %zu", pc.why, line, col + 1);
        }
    }
    std::vector<size_t> total(spans.size(), 0);
    for (const Piece &pc : pieces) total[pc.span] += pc.out.size();
    for (size_t s = 0; s < spans.size(); ++s) sd->entries[spans[s].entry].data.resize(total[s]);
    std::vector<size_t> offset(pieces.size(), 0);
    {
        std::vector<size_t> run(spans.size(), 0);
        for (size_t i = 0; i < pieces.size(); ++i) {
            offset[i] = run[pieces[i].span];
            run[pieces[i].span] += pieces[i].out.size();
        }
    }
    parallel_for(pieces.size(), [&](size_t i) {
        Piece &pc = pieces[i];
        if (!pc.out.empty())
            memcpy(sd->entries[spans[pc.span].entry].data.data() + offset[i], pc.out.data(),
                   pc.out.size() * sizeof(float));
        std::vector<float>().swap(pc.out);
    });
    std::sort(sd->entries.begin(), sd->entries.end(),
              [](const m3_state_dict::Entry &a, const m3_state_dict::Entry &b) { return a.name < b.name; });
    *out = sd;
    return m3::api_ok();
}

// ---------------------------------------------------------------- writer
void put_json_string(std::string &o, const char *s) {
    o += '"';
    for (const unsigned char *q = reinterpret_cast<const unsigned char *>(s); *q; ++q) {
        const unsigned char c = *q;
        if (c == '"') o += "\\\"";
        else if (c == '\\') o += "\\\\";
        else if (c == '\n') o += "\\n";
        else if (c == '\r') o += "\\r";
        else if (c == '\t') o += "\\t";
        else if (c == '\b') o += "\\b";
        else if (c == '\f') o += "\\f";
        else if (c < 0x20) {
            char buf[8];
            snprintf(buf, sizeof(buf), "\\u%04x", c);
            o += buf;
        } else {
            o += static_cast<char>(c);
        }
    }
    o += '"';
}

void put_floats(std::string &o, const float *v, size_t n) {
    char buf[32];
    for (size_t i = 0; i < n; ++i) {
        if (i) o += ',';
        if (!std::isfinite(v[i])) {
            o += "null";
            continue;
        }
        const auto r = std::to_chars(buf, buf + sizeof(buf), v[i]);
        o.append(buf, r.ptr);
    }
}

}  // namespace

extern "C" {

m3_status m3_checkpoint_load(const char *path, m3_state_dict **out) { return load(path, true, out); }

m3_status m3_state_dict_load(const char *path, m3_state_dict **out) { return load(path, false, out); }

void m3_state_dict_free(m3_state_dict *sd) { delete sd; }

size_t m3_state_dict_len(const m3_state_dict *sd) { return sd ? sd->entries.size() : 0; }

m3_status m3_state_dict_entry(const m3_state_dict *sd, size_t index, const char **name,
                              size_t *ndim, const size_t **shape, const float **data,
                              size_t *numel) {
    if (sd == nullptr) return m3::api_fail(M3_ERR_ARGUMENT, "state dict is NULL");
    if (index >= sd->entries.size())
        return m3::api_fail(M3_ERR_ARGUMENT, "entry %zu of %zu", index, sd->entries.size());
    const auto &e = sd->entries[index];
    if (name) *name = e.name.c_str();
    if (ndim) *ndim = e.shape.size();
    if (shape) *shape = e.shape.data();
    if (data) *data = e.data.data();
    if (numel) *numel = e.data.size();
    return m3::api_ok();
}

int64_t m3_state_dict_find(const m3_state_dict *sd, const char *name) {
    if (sd == nullptr || name == nullptr) return -1;
    const auto it = std::lower_bound(
        sd->entries.begin(), sd->entries.end(), name,
        [](const m3_state_dict::Entry &e, const char *n) { return e.name < n; });
    if (it == sd->entries.end() || it->name != name) return -1;
    return static_cast<int64_t>(it - sd->entries.begin());
}

uint64_t m3_checkpoint_step(const m3_state_dict *sd) { return sd ? sd->step : 0; }

const char *m3_checkpoint_metadata(const m3_state_dict *sd) { return sd ? sd->metadata.c_str() : "null"; }

m3_status m3_state_dict_save(const char *path, int32_t as_checkpoint, uint64_t step,
                             const char *metadata_json, size_t n, const char *const *names,
                             const size_t *ndims, const size_t *const *shapes,
                             const float *const *data, const size_t *numels) {
    if (path == nullptr) return m3::api_fail(M3_ERR_ARGUMENT, "path is NULL");
    if (n > 0 && (names == nullptr || ndims == nullptr || shapes == nullptr || data == nullptr ||
                  numels == nullptr))
        return m3::api_fail(M3_ERR_ARGUMENT, "entry arrays are NULL");
    std::string meta = metadata_json ? metadata_json : "null";
    if (as_checkpoint) {
        Parser check(meta.data(), meta.size());
        if (!check.whole_value()) return m3::api_fail(M3_ERR_ARGUMENT, "metadata is not valid JSON");
    }
    std::vector<size_t> order(n);
    for (size_t i = 0; i < n; ++i) {
        if (names[i] == nullptr) return m3::api_fail(M3_ERR_ARGUMENT, "entry %zu has no name", i);
        if (numels[i] > 0 && data[i] == nullptr)
            return m3::api_fail(M3_ERR_ARGUMENT, "entry `%s` has no data", names[i]);
        if (ndims[i] > 0 && shapes[i] == nullptr)
            return m3::api_fail(M3_ERR_ARGUMENT, "entry `%s` has no shape", names[i]);
        order[i] = i;
    }
    std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return strcmp(names[a], names[b]) < 0; });
    for (size_t i = 1; i < n; ++i)
        if (strcmp(names[order[i - 1]], names[order[i]]) == 0)
            return m3::api_fail(M3_ERR_ARGUMENT, "entry `%s` appears twice", names[order[i]]);
    // format each entry's numbers in parallel pieces, then write in order
    struct Chunk {
        size_t entry, begin, count;
        std::string text;
    };
    std::vector<Chunk> chunks;
    constexpr size_t kValues = size_t(1) << 19;
    for (size_t k = 0; k < n; ++k) {
        const size_t i = order[k];
        size_t b = 0;
        do {
            const size_t c = std::min(kValues, numels[i] - b);
            chunks.push_back(Chunk{i, b, c, std::string()});
            b += c;
        } while (b < numels[i]);
    }
    parallel_for(chunks.size(), [&](size_t j) {
        Chunk &c = chunks[j];
        c.text.reserve(c.count * 12);
        put_floats(c.text, data[c.entry] + c.begin, c.count);
    });
    FILE *f = fopen(path, "wb");
    if (f == nullptr) return m3::api_fail(M3_ERR_IO, "%s: %s", path, strerror(errno));
    std::string head;
    if (as_checkpoint) head = "{\"step\":" + std::to_string(step) + ",\"state\":";
    head += "{\"entries\":{";
    bool okw = fwrite(head.data(), 1, head.size(), f) == head.size();
    size_t j = 0;
    for (size_t k = 0; k < n && okw; ++k) {
        const size_t i = order[k];
        std::string pre;
        if (k) pre += ',';
        put_json_string(pre, names[i]);
        pre += ":{\"shape\":[";
        for (size_t d = 0; d < ndims[i]; ++d) {
            if (d) pre += ',';
            pre += std::to_string(shapes[i][d]);
        }
        pre += "],\"data\":[";
        okw = fwrite(pre.data(), 1, pre.size(), f) == pre.size();
        bool first = true;
        for (; okw && j < chunks.size() && chunks[j].entry == i; ++j) {
            if (chunks[j].count == 0) continue;
            if (!first) okw = fputc(',', f) != EOF;
            first = false;
            okw = okw && fwrite(chunks[j].text.data(), 1, chunks[j].text.size(), f) == chunks[j].text.size();
        }
        okw = okw && fwrite("]}", 1, 2, f) == 2;
    }
    std::string tail = "}}";
    if (as_checkpoint) tail += ",\"metadata\":" + meta + "}";
    okw = okw && fwrite(tail.data(), 1, tail.size(), f) == tail.size();
    const bool closed = fclose(f) == 0;
    if (!okw || !closed) return m3::api_fail(M3_ERR_IO, "%s: write failed", path);
    return m3::api_ok();
}

}  // extern "C"
