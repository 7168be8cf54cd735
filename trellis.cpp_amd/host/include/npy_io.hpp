// Minimal .npy (format 1.0 / 2.0) reader and writer for the host check programs and the decoder
// benchmark: C-order little-endian float32 ('<f4'), int32 ('<i4') and uint8 ('|u1') arrays.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstring>
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

inline Array load(const std::string& path) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) throw std::runtime_error("cannot open " + path);
    char magic[8];
    if (fread(magic, 1, 8, f) != 8 || memcmp(magic, "\x93NUMPY", 6) != 0) {
        fclose(f);
        throw std::runtime_error(path + ": not a .npy file");
    }
    uint32_t hlen = 0;
    if (magic[6] == 1) {
        uint16_t h16;
        if (fread(&h16, 2, 1, f) != 1) { fclose(f); throw std::runtime_error(path + ": truncated"); }
        hlen = h16;
    } else if (fread(&hlen, 4, 1, f) != 1) {
        fclose(f);
        throw std::runtime_error(path + ": truncated");
    }
    std::string h(hlen, ' ');
    if (fread(&h[0], 1, hlen, f) != hlen) { fclose(f); throw std::runtime_error(path + ": truncated"); }
    Array a;
    auto field = [&](const char* key) {
        const size_t p = h.find(key);
        if (p == std::string::npos) throw std::runtime_error(path + ": header lacks " + key);
        return h.find(':', p) + 1;
    };
    size_t p = h.find('\'', field("'descr'"));
    a.descr = h.substr(p + 1, h.find('\'', p + 1) - p - 1);
    if (h.find("True", field("'fortran_order'")) < h.find(',', field("'fortran_order'")))
        throw std::runtime_error(path + ": Fortran order not supported");
    p = h.find('(', field("'shape'"));
    const size_t e = h.find(')', p);
    std::string dims = h.substr(p + 1, e - p - 1);
    size_t q = 0;
    while (q < dims.size()) {
        while (q < dims.size() && (dims[q] == ' ' || dims[q] == ',')) ++q;
        if (q >= dims.size()) break;
        a.shape.push_back(std::stoll(dims.substr(q)));
        while (q < dims.size() && dims[q] != ',') ++q;
    }
    size_t es = 0;
    if (a.descr == "<f4" || a.descr == "<i4") es = 4;
    else if (a.descr == "|u1" || a.descr == "<u1") es = 1;
    else { fclose(f); throw std::runtime_error(path + ": dtype " + a.descr + " not supported"); }
    a.bytes.resize((size_t)a.size() * es);
    if (!a.bytes.empty() && fread(a.bytes.data(), 1, a.bytes.size(), f) != a.bytes.size()) {
        fclose(f);
        throw std::runtime_error(path + ": truncated data");
    }
    fclose(f);
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
