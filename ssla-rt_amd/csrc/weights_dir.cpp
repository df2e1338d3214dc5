// weights_dir.cpp -- weights.npz (stored ZIP of .npy members) and meta.json
// reader.  Host code only; see weights_dir.h.
//
// The ZIP walk goes through the central directory (PKWARE APPNOTE 4.3.12,
// 4.3.16) so it does not depend on local-header sizes; ZIP64 sizes and
// offsets (extra field 0x0001, APPNOTE 4.5.3) are honoured.  Each member is
// a NumPy .npy file (format versions 1.0 - 3.0) holding '<f4' C-order data.
#include "weights_dir.h"

#include <cctype>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>
#include <stdexcept>

namespace ssla {
namespace {

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error(what); }

std::string slurp(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) fail("cannot open " + path);
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

uint64_t le(const std::string& b, size_t off, int n) {
    if (off + n > b.size()) fail("truncated zip structure");
    uint64_t v = 0;
    for (int i = n - 1; i >= 0; --i) v = (v << 8) | static_cast<uint8_t>(b[off + i]);
    return v;
}

// ---- .npy ---------------------------------------------------------------

// Finds the value text of `'key':` inside a Python dict literal header.
std::string dict_value(const std::string& hdr, const std::string& key) {
    const std::string pat = "'" + key + "'";
    size_t p = hdr.find(pat);
    if (p == std::string::npos) fail("npy header lacks " + key);
    p = hdr.find(':', p + pat.size());
    if (p == std::string::npos) fail("npy header malformed at " + key);
    ++p;
    while (p < hdr.size() && hdr[p] == ' ') ++p;
    size_t e = p;
    if (e < hdr.size() && hdr[e] == '(') {
        e = hdr.find(')', e);
        if (e == std::string::npos) fail("npy shape malformed");
        return hdr.substr(p, e - p + 1);
    }
    while (e < hdr.size() && hdr[e] != ',' && hdr[e] != '}') ++e;
    return hdr.substr(p, e - p);
}

NpzTensor parse_npy(const char* d, size_t n, const std::string& name) {
    static const char magic[] = "\x93NUMPY";
    if (n < 10 || std::memcmp(d, magic, 6) != 0) fail(name + ": not an .npy member");
    const int major = static_cast<uint8_t>(d[6]);
    size_t hlen, hoff;
    if (major == 1) {
        hlen = static_cast<uint8_t>(d[8]) | (static_cast<size_t>(static_cast<uint8_t>(d[9])) << 8);
        hoff = 10;
    } else if (major == 2 || major == 3) {
        if (n < 12) fail(name + ": truncated npy header");
        hlen = 0;
        for (int i = 3; i >= 0; --i) hlen = (hlen << 8) | static_cast<uint8_t>(d[8 + i]);
        hoff = 12;
    } else {
        fail(name + ": unsupported npy version");
    }
    if (hoff + hlen > n) fail(name + ": truncated npy header");
    const std::string hdr(d + hoff, hlen);
    const std::string descr = dict_value(hdr, "descr");
    if (descr.find("<f4") == std::string::npos)
        fail(name + ": dtype " + descr + " is not '<f4'");
    if (dict_value(hdr, "fortran_order").find("False") == std::string::npos)
        fail(name + ": fortran_order arrays are not supported");
    const std::string shp = dict_value(hdr, "shape");
    NpzTensor t;
    size_t i = 1;
    while (i < shp.size()) {
        while (i < shp.size() && (shp[i] == ' ' || shp[i] == ',')) ++i;
        if (i >= shp.size() || shp[i] == ')') break;
        size_t j = i;
        while (j < shp.size() && shp[j] >= '0' && shp[j] <= '9') ++j;
        if (j == i) fail(name + ": bad shape " + shp);
        t.shape.push_back(std::stoll(shp.substr(i, j - i)));
        i = j;
    }
    const size_t body = hoff + hlen;
    const int64_t cnt = t.numel();
    if (cnt < 0 || body + static_cast<size_t>(cnt) * 4 > n) fail(name + ": payload shorter than shape");
    t.data.resize(static_cast<size_t>(cnt));
    if (cnt) std::memcpy(t.data.data(), d + body, static_cast<size_t>(cnt) * 4);
    return t;
}

// ---- json (flat object of strings and numbers) ---------------------------

std::map<std::string, std::string> parse_flat_json(const std::string& s,
                                                   const std::string& path) {
    std::map<std::string, std::string> out;
    size_t p = s.find('{');
    if (p == std::string::npos) fail(path + ": not a JSON object");
    ++p;
    auto skip = [&]() { while (p < s.size() && std::isspace(static_cast<unsigned char>(s[p]))) ++p; };
    auto read_string = [&]() {
        if (s[p] != '"') fail(path + ": expected string");
        std::string v;
        ++p;
        while (p < s.size() && s[p] != '"') {
            if (s[p] == '\\' && p + 1 < s.size()) ++p;
            v += s[p++];
        }
        if (p >= s.size()) fail(path + ": unterminated string");
        ++p;
        return v;
    };
    while (true) {
        skip();
        if (p >= s.size()) fail(path + ": unterminated object");
        if (s[p] == '}') break;
        const std::string key = read_string();
        skip();
        if (p >= s.size() || s[p] != ':') fail(path + ": expected ':' after " + key);
        ++p;
        skip();
        std::string val;
        if (s[p] == '"') {
            val = read_string();
        } else {
            int depth = 0;
            size_t b = p;
            while (p < s.size()) {
                const char c = s[p];
                if (c == '[' || c == '{') ++depth;
                else if (c == ']' || c == '}') { if (depth == 0) break; --depth; }
                else if (c == ',' && depth == 0) break;
                ++p;
            }
            val = s.substr(b, p - b);
            while (!val.empty() && std::isspace(static_cast<unsigned char>(val.back()))) val.pop_back();
        }
        out[key] = val;
        skip();
        if (p < s.size() && s[p] == ',') ++p;
    }
    return out;
}

int to_int(const std::map<std::string, std::string>& m, const char* k, int dflt) {
    const auto it = m.find(k);
    if (it == m.end()) return dflt;
    try { return std::stoi(it->second); } catch (...) { fail(std::string("meta.json: bad integer for ") + k); }
}

}  // namespace

ModelMeta read_meta(const std::string& dir) {
    const std::string path = dir + "/meta.json";
    const auto kv = parse_flat_json(slurp(path), path);
    ModelMeta m;
    m.schema_version = to_int(kv, "schema_version", 0);
    const auto it = kv.find("model");
    if (it != kv.end()) m.model = it->second;
    m.height = to_int(kv, "height", 0);
    m.width = to_int(kv, "width", 0);
    m.num_classes = to_int(kv, "num_classes", 0);
    m.ssla_tdrop_window = to_int(kv, "ssla_tdrop_window", 0);
    if (m.schema_version != 1)
        fail(path + ": schema_version " + std::to_string(m.schema_version) + " unsupported");
    return m;
}

std::map<std::string, NpzTensor> read_npz(const std::string& dir) {
    const std::string path = dir + "/weights.npz";
    const std::string b = slurp(path);
    // End of central directory record: last occurrence of PK\5\6.
    if (b.size() < 22) fail(path + ": too small for a zip archive");
    size_t eocd = std::string::npos;
    const size_t lo = b.size() > 65557 ? b.size() - 65557 : 0;
    for (size_t i = b.size() - 22 + 1; i-- > lo;) {
        if (le(b, i, 4) == 0x06054b50u) { eocd = i; break; }
    }
    if (eocd == std::string::npos) fail(path + ": no end-of-central-directory record");
    uint64_t n_entries = le(b, eocd + 10, 2);
    uint64_t cd_off = le(b, eocd + 16, 4);
    if (n_entries == 0xFFFF || cd_off == 0xFFFFFFFFu) {
        // ZIP64 end of central directory locator sits right before the EOCD.
        if (eocd < 20 || le(b, eocd - 20, 4) != 0x07064b50u) fail(path + ": missing ZIP64 locator");
        const uint64_t z64 = le(b, eocd - 20 + 8, 8);
        if (le(b, z64, 4) != 0x06064b50u) fail(path + ": bad ZIP64 end record");
        n_entries = le(b, z64 + 32, 8);
        cd_off = le(b, z64 + 48, 8);
    }
    std::map<std::string, NpzTensor> out;
    size_t p = cd_off;
    for (uint64_t e = 0; e < n_entries; ++e) {
        if (le(b, p, 4) != 0x02014b50u) fail(path + ": bad central directory entry");
        const uint64_t method = le(b, p + 10, 2);
        uint64_t csize = le(b, p + 20, 4);
        uint64_t usize = le(b, p + 24, 4);
        const uint64_t nlen = le(b, p + 28, 2), xlen = le(b, p + 30, 2), clen = le(b, p + 32, 2);
        uint64_t loff = le(b, p + 42, 4);
        std::string name = b.substr(p + 46, nlen);
        // ZIP64 extended information: fields present only for saturated values.
        size_t x = p + 46 + nlen;
        const size_t xend = x + xlen;
        while (x + 4 <= xend) {
            const uint64_t id = le(b, x, 2), sz = le(b, x + 2, 2);
            if (id == 0x0001) {
                size_t q = x + 4;
                if (usize == 0xFFFFFFFFu) { usize = le(b, q, 8); q += 8; }
                if (csize == 0xFFFFFFFFu) { csize = le(b, q, 8); q += 8; }
                if (loff == 0xFFFFFFFFu) { loff = le(b, q, 8); q += 8; }
            }
            x += 4 + sz;
        }
        p = xend + clen;
        if (method != 0) fail(path + ": member " + name + " is compressed (np.savez_compressed is unsupported)");
        if (csize != usize) fail(path + ": member " + name + " size mismatch");
        if (le(b, loff, 4) != 0x04034b50u) fail(path + ": bad local header for " + name);
        const uint64_t data = loff + 30 + le(b, loff + 26, 2) + le(b, loff + 28, 2);
        if (data + csize > b.size()) fail(path + ": member " + name + " runs past end of file");
        if (name.size() > 4 && name.compare(name.size() - 4, 4, ".npy") == 0) name.resize(name.size() - 4);
        out[name] = parse_npy(b.data() + data, static_cast<size_t>(csize), path + ":" + name);
    }
    return out;
}

}  // namespace ssla
