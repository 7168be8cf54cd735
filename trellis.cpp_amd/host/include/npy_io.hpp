// Minimal .npy (format 1.0 / 2.0) reader and writer for the host check programs and the decoder
// benchmark: C-order little-endian float32 ('<f4'), int32 ('<i4') and uint8 ('|u1') arrays.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace npyio {

struct Array {
    std::string descr;
    std::vector<int64_t> shape;
    std::vector<uint8_t> bytes;
    int64_t size() const {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        return n;
    }
    template <class T> const T* as() const { return reinterpret_cast<const T*>(bytes.data()); }
};

// Reads a C-order .npy file of dtype <f4, <i4 or |u1. Throws std::runtime_error for anything
// else, including a header or shape that does not parse or data shorter than the shape.
inline Array load(const std::string& path) {
    struct Closer {
        void operator()(FILE* f) const { fclose(f); }
    };
    std::unique_ptr<FILE, Closer> file(fopen(path.c_str(), "rb"));
    FILE* f = file.get();
    if (!f) throw std::runtime_error("cannot open " + path);
    auto fail = [&](const std::string& why) { return std::runtime_error(path + ": " + why); };
    if (fseek(f, 0, SEEK_END) != 0) throw fail("cannot seek");
    const long fsize = ftell(f);
    rewind(f);
    char magic[8];
    if (fread(magic, 1, 8, f) != 8 || memcmp(magic, "\x93NUMPY", 6) != 0) throw fail("not a .npy file");
    uint32_t hlen = 0;
    if (magic[6] == 1) {
        uint16_t h16;
        if (fread(&h16, 2, 1, f) != 1) throw fail("truncated");
        hlen = h16;
    } else if (fread(&hlen, 4, 1, f) != 1) {
        throw fail("truncated");
    }
    if ((long)hlen > fsize) throw fail("truncated");
    std::string h(hlen, ' ');
    if (hlen && fread(&h[0], 1, hlen, f) != hlen) throw fail("truncated");
    Array a;
    // the position just after "key":, or a parse error
    auto field = [&](const char* key) {
        const size_t p = h.find(key);
        if (p == std::string::npos) throw fail(std::string("header lacks ") + key);
        const size_t c = h.find(':', p);
        if (c == std::string::npos) throw fail(std::string("header lacks a value for ") + key);
        return c + 1;
    };
    const size_t d0 = h.find('\'', field("'descr'"));
    const size_t d1 = d0 == std::string::npos ? d0 : h.find('\'', d0 + 1);
    if (d1 == std::string::npos) throw fail("bad descr");
    a.descr = h.substr(d0 + 1, d1 - d0 - 1);
    const size_t fo = field("'fortran_order'");
    if (h.find("True", fo) < h.find(',', fo)) throw fail("Fortran order not supported");
    const size_t s0 = h.find('(', field("'shape'"));
    const size_t s1 = s0 == std::string::npos ? s0 : h.find(')', s0);
    if (s1 == std::string::npos) throw fail("bad shape");
    const std::string dims = h.substr(s0 + 1, s1 - s0 - 1);
    size_t q = 0;
    while (q < dims.size()) {
        while (q < dims.size() && (dims[q] == ' ' || dims[q] == ',')) ++q;
        if (q >= dims.size()) break;
        size_t used = 0;
        long long d = -1;
        try {
            d = std::stoll(dims.substr(q), &used);
        } catch (const std::exception&) {
            throw fail("bad shape");
        }
        if (d < 0 || used == 0) throw fail("bad shape");
        a.shape.push_back(d);
        q += used;
        while (q < dims.size() && dims[q] != ',') ++q;
    }
    size_t es = 0;
    if (a.descr == "<f4" || a.descr == "<i4") es = 4;
    else if (a.descr == "|u1" || a.descr == "<u1") es = 1;
    else throw fail("dtype " + a.descr + " not supported");
    // the element count, checked against the bytes left in the file before anything is allocated
    const uint64_t left = (uint64_t)(fsize - ftell(f));
    uint64_t count = 1;
    for (int64_t d : a.shape) {
        if (d != 0 && count > left / (uint64_t)d) throw fail("truncated data");
        count *= (uint64_t)d;
    }
    if (count > left / es) throw fail("truncated data");
    a.bytes.resize((size_t)(count * es));
    if (!a.bytes.empty() && fread(a.bytes.data(), 1, a.bytes.size(), f) != a.bytes.size()) throw fail("truncated data");
    return a;
}

inline void save(const std::string& path, const char* descr, const std::vector<int64_t>& shape,
                 const void* data, size_t nbytes) {
    std::string dims;
    for (int64_t d : shape) dims += std::to_string(d) + ",";
    if (shape.size() > 1) dims.pop_back();
    std::string h = std::string("{'descr': '") + descr + "', 'fortran_order': False, 'shape': (" + dims + "), }";
    while ((10 + h.size() + 1) % 64) h += ' ';
    h += '\n';
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) throw std::runtime_error("cannot write " + path);
    const uint16_t hl = (uint16_t)h.size();
    fwrite("\x93NUMPY\x01\x00", 1, 8, f);
    fwrite(&hl, 2, 1, f);
    fwrite(h.data(), 1, h.size(), f);
    if (nbytes) fwrite(data, 1, nbytes, f);
    fclose(f);
}

}  // namespace npyio
