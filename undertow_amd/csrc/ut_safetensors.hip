// ut_safetensors.hip -- safetensors headers and shard index (host code):
// a small JSON reader, header validation and pread.
#include "ut_safetensors.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <limits>

namespace ut {
namespace st {

namespace {

struct Parser {
    const char *p, *end;
    std::string err;
    int depth = 0;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    bool fail(const char *what) {
        if (err.empty()) err = what;
        return false;
    }
    static void utf8(std::string &s, uint32_t c) {
        if (c < 0x80) {
            s += (char)c;
        } else if (c < 0x800) {
            s += (char)(0xC0 | (c >> 6));
            s += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            s += (char)(0xE0 | (c >> 12));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        } else {
            s += (char)(0xF0 | (c >> 18));
            s += (char)(0x80 | ((c >> 12) & 0x3F));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t &v) {
        if (end - p < 4) return fail("short \\u escape");
        v = 0;
        for (int k = 0; k < 4; k++) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool str(std::string &s) {
        if (p >= end || *p != '"') return fail("expected a string");
        p++;
        while (p < end && *p != '"') {
            const unsigned char c = (unsigned char)*p++;
            if (c < 0x20) return fail("control character in a string");
            if (c != '\\') {
                s += (char)c;
                continue;
            }
            if (p >= end) return fail("unterminated escape");
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
                uint32_t v;
                if (!hex4(v)) return false;
                if (v >= 0xD800 && v < 0xDC00) {
                    uint32_t lo;
                    if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return fail("lone surrogate");
                    p += 2;
                    if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
                    v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(s, v);
                break;
            }
            default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool num(Json &v) {
        const char *s0 = p;
        bool neg = false, frac = false;
        if (p < end && *p == '-') { neg = true; p++; }
        if (p >= end || *p < '0' || *p > '9') return fail("bad number");
        uint64_t acc = 0;
        bool over = false;
        while (p < end && *p >= '0' && *p <= '9') {
            const uint64_t dgt = (uint64_t)(*p++ - '0');
            if (acc > (std::numeric_limits<uint64_t>::max() - dgt) / 10) over = true;
            acc = acc * 10 + dgt;
        }
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) {
            frac = true;
            while (p < end && (*p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-' ||
                               (*p >= '0' && *p <= '9')))
                p++;
        }
        if (frac || over || acc > (uint64_t)std::numeric_limits<int64_t>::max()) {
            v.kind = Json::Num;
            v.d = strtod(std::string(s0, p).c_str(), nullptr);
        } else {
            v.kind = Json::Int;
            v.i = neg ? -(int64_t)acc : (int64_t)acc;
            v.d = (double)v.i;
        }
        return true;
    }
    bool lit(const char *w) {
        const size_t n = strlen(w);
        if ((size_t)(end - p) < n || memcmp(p, w, n) != 0) return fail("bad literal");
        p += n;
        return true;
    }
    bool value(Json &v) {
        if (++depth > 64) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end");
        bool ok = true;
        const char c = *p;
        if (c == '{') {
            v.kind = Json::Obj;
            p++;
            ws();
            if (p < end && *p == '}') {
                p++;
            } else {
                for (;;) {
                    ws();
                    std::string k;
                    Json x;
                    if (!str(k)) { ok = false; break; }
                    ws();
                    if (p >= end || *p != ':') { ok = fail("expected ':'"); break; }
                    p++;
                    if (!value(x)) { ok = false; break; }
                    v.obj.emplace_back(std::move(k), std::move(x));
                    ws();
                    if (p < end && *p == ',') { p++; continue; }
                    if (p < end && *p == '}') { p++; break; }
                    ok = fail("expected ',' or '}'");
                    break;
                }
            }
        } else if (c == '[') {
            v.kind = Json::Arr;
            p++;
            ws();
            if (p < end && *p == ']') {
                p++;
            } else {
                for (;;) {
                    Json x;
                    if (!value(x)) { ok = false; break; }
                    v.arr.push_back(std::move(x));
                    ws();
                    if (p < end && *p == ',') { p++; continue; }
                    if (p < end && *p == ']') { p++; break; }
                    ok = fail("expected ',' or ']'");
                    break;
                }
            }
        } else if (c == '"') {
            v.kind = Json::Str;
            ok = str(v.s);
        } else if (c == 't') {
            v.kind = Json::Bool;
            v.b = true;
            ok = lit("true");
        } else if (c == 'f') {
            v.kind = Json::Bool;
            ok = lit("false");
        } else if (c == 'n') {
            ok = lit("null");
        } else {
            ok = num(v);
        }
        depth--;
        return ok;
    }
};

bool parse_dtype(const std::string &s, int &d) {
    if (s == "F32") d = ST_F32;
    else if (s == "F16") d = ST_F16;
    else if (s == "BF16") d = ST_BF16;
    else if (s == "U8") d = ST_U8;
    else if (s == "I8") d = ST_I8;
    else return false;
    return true;
}

bool read_file(const std::string &path, std::string &out, std::string &err) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        err = path + ": " + strerror(errno);
        return false;
    }
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        err = path + ": " + strerror(errno);
        ::close(fd);
        return false;
    }
    out.resize((size_t)sb.st_size);
    Shard s{path, fd, (uint64_t)sb.st_size};
    const bool ok = read_at(s, &out[0], (uint64_t)sb.st_size, 0, err);
    ::close(fd);
    return ok;
}

// SafetensorsReader::open + parse_header (reader.rs:78-143, 150-185).
bool open_shard(const std::string &path, int shard_no, Index &idx,
                std::unordered_map<std::string, Entry> &out, std::string &err) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        err = path + ": " + strerror(errno);
        return false;
    }
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        err = path + ": " + strerror(errno);
        ::close(fd);
        return false;
    }
    idx.shards.push_back({path, fd, (uint64_t)sb.st_size});
    const Shard &s = idx.shards.back();
    uint8_t lb[8];
    if (!read_at(s, lb, 8, 0, err)) return false;
    uint64_t hl = 0;
    for (int i = 0; i < 8; i++) hl |= (uint64_t)lb[i] << (8 * i);
    if (hl > (uint64_t)100 * 1024 * 1024) {
        err = path + ": safetensors header length " + std::to_string(hl) + " exceeds limit";
        return false;
    }
    if (8 + hl > s.file_len) {
        err = path + ": header runs past the end of the file";
        return false;
    }
    std::string hdr((size_t)hl, '\0');
    if (hl && !read_at(s, &hdr[0], hl, 8, err)) return false;
    Json root;
    std::string jerr;
    if (!parse_json(hdr.data(), hdr.size(), root, jerr)) {
        err = path + ": bad header json: " + jerr;
        return false;
    }
    if (root.kind != Json::Obj) {
        err = path + ": header is not an object";
        return false;
    }
    const uint64_t data_start = 8 + hl;
    for (auto &kv : root.obj) {
        const std::string &name = kv.first;
        if (name == "__metadata__") continue;
        const Json &v = kv.second;
        const std::string bad = path + ": bad entry for " + name;
        const Json *dt = v.get("dtype"), *sh = v.get("shape"), *of = v.get("data_offsets");
        Entry e;
        if (!dt || dt->kind != Json::Str || !parse_dtype(dt->s, e.dtype)) {
            err = dt && dt->kind == Json::Str ? path + ": unsupported safetensors dtype: " + dt->s : bad;
            return false;
        }
        if (!sh || sh->kind != Json::Arr || !of || of->kind != Json::Arr || of->arr.size() != 2) {
            err = bad;
            return false;
        }
        uint64_t expected = (uint64_t)dtype_size(e.dtype);
        for (auto &d : sh->arr) {
            if (d.kind != Json::Int || d.i < 0) {
                err = bad;
                return false;
            }
            e.shape.push_back(d.i);
            if (d.i != 0 && expected > std::numeric_limits<uint64_t>::max() / (uint64_t)d.i) {
                err = bad;
                return false;
            }
            expected *= (uint64_t)d.i;
        }
        const Json &a = of->arr[0], &b = of->arr[1];
        if (a.kind != Json::Int || b.kind != Json::Int || a.i < 0 || b.i < a.i) {
            err = bad;
            return false;
        }
        const uint64_t start = (uint64_t)a.i, stop = (uint64_t)b.i;
        if (stop - start != expected || data_start + stop > s.file_len || data_start + stop < data_start) {
            err = path + ": tensor " + name + " offsets inconsistent with shape/dtype/file size";
            return false;
        }
        e.offset = data_start + start;
        e.nbytes = stop - start;
        e.shard = shard_no;
        out[name] = std::move(e);
    }
    return true;
}

}  // namespace

bool parse_json(const char *text, size_t n, Json &out, std::string &err) {
    Parser ps{text, text + n, {}};
    if (!ps.value(out)) {
        err = ps.err;
        return false;
    }
    ps.ws();
    if (ps.p != ps.end) {
        err = "trailing characters";
        return false;
    }
    return true;
}

bool read_at(const Shard &s, void *dst, uint64_t n, uint64_t offset, std::string &err) {
    char *d = (char *)dst;
    while (n > 0) {
        const size_t want = n > ((uint64_t)1 << 30) ? ((size_t)1 << 30) : (size_t)n;
        const ssize_t r = ::pread(s.fd, d, want, (off_t)offset);
        if (r < 0) {
            if (errno == EINTR) continue;
            err = s.path + ": " + strerror(errno);
            return false;
        }
        if (r == 0) {
            err = s.path + ": unexpected end of file";
            return false;
        }
        d += r;
        n -= (uint64_t)r;
        offset += (uint64_t)r;
    }
    return true;
}

void widen_halves(const uint16_t *src, uint64_t n, bool bf16, uint32_t *dst) {
    for (uint64_t i = 0; i < n; i++) {
        const uint32_t h = src[i];
        if (bf16) {
            dst[i] = h << 16;
            continue;
        }
        // IEEE binary16 -> binary32
        const uint32_t sign = (h & 0x8000u) << 16, ex = (h >> 10) & 0x1F, man = h & 0x3FF;
        uint32_t v;
        if (ex == 0x1F) {
            v = sign | 0x7F800000u | (man << 13);
        } else if (ex != 0) {
            v = sign | ((ex + 112) << 23) | (man << 13);
        } else if (man == 0) {
            v = sign;
        } else {
            int e = -1;
            uint32_t m = man;
            do { e++; m <<= 1; } while (!(m & 0x400));
            v = sign | ((uint32_t)(112 - e) << 23) | ((m & 0x3FF) << 13);
        }
        dst[i] = v;
    }
}

bool read_f32_at(const Shard &s, const Entry &e, float *dst, std::vector<uint16_t> &tmp,
                 std::string &err) {
    if (e.dtype == ST_F32) return read_at(s, dst, e.nbytes, e.offset, err);
    if (e.dtype != ST_BF16 && e.dtype != ST_F16) {
        err = s.path + ": cannot convert the tensor to f32";
        return false;
    }
    const uint64_t n = e.nbytes / 2;
    tmp.resize((size_t)n);
    if (!read_at(s, tmp.data(), e.nbytes, e.offset, err)) return false;
    widen_halves(tmp.data(), n, e.dtype == ST_BF16, (uint32_t *)dst);
    return true;
}

Index::~Index() {
    for (auto &s : shards)
        if (s.fd >= 0) ::close(s.fd);
}

bool open_dir(const std::string &dir, Index &idx, std::string &err) {
    const std::string index_path = dir + "/model.safetensors.index.json";
    struct stat sb;
    if (stat(index_path.c_str(), &sb) == 0) {
        std::string text;
        if (!read_file(index_path, text, err)) return false;
        Json root;
        std::string jerr;
        if (!parse_json(text.data(), text.size(), root, jerr)) {
            err = index_path + ": bad index json: " + jerr;
            return false;
        }
        const Json *wm = root.kind == Json::Obj ? root.get("weight_map") : nullptr;
        if (!wm || wm->kind != Json::Obj) {
            err = index_path + ": missing weight_map";
            return false;
        }
        std::unordered_map<std::string, int> shard_ids;
        std::vector<std::unordered_map<std::string, Entry>> per;  // each shard's entries
        for (auto &kv : wm->obj) {
            if (kv.second.kind != Json::Str) {
                err = index_path + ": bad weight_map entry";
                return false;
            }
            const std::string &file = kv.second.s;
            if (file.find('/') != std::string::npos || file == ".." || file.empty()) {
                err = index_path + ": shard name " + file + " leaves the model directory";
                return false;
            }
            auto it = shard_ids.find(file);
            int id;
            if (it == shard_ids.end()) {
                id = (int)idx.shards.size();
                per.emplace_back();
                if (!open_shard(dir + "/" + file, id, idx, per.back(), err)) return false;
                shard_ids.emplace(file, id);
            } else {
                id = it->second;
            }
            // the index names each tensor's shard: take the entry from there
            auto e = per[(size_t)id].find(kv.first);
            if (e == per[(size_t)id].end()) {
                err = index_path + ": " + kv.first + " is not in " + file;
                return false;
            }
            idx.tensors[kv.first] = e->second;
        }
        return true;
    }
    return open_shard(dir + "/model.safetensors", 0, idx, idx.tensors, err);
}

}  // namespace st
}  // namespace ut
