#include "sbb_reader.h"

#include <stdio.h>
#include <string.h>

namespace sbh {

static uint32_t rd32(const unsigned char* p) { uint32_t v; memcpy(&v, p, 4); return v; }
static uint64_t rd64(const unsigned char* p) { uint64_t v; memcpy(&v, p, 8); return v; }

bool Blob::open(const std::string& path, std::string* err) {
    path_ = path;
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) { *err = "cannot open " + path; return false; }
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (sz < 52) { fclose(f); *err = "truncated blob " + path; return false; }
    // 8-byte aligned storage; sections are 64-aligned relative to the file start
    buf_.assign((size_t)sz + 64, 0);
    size_t shift = (64 - ((uintptr_t)buf_.data() & 63)) & 63;
    unsigned char* m = buf_.data() + shift;
    if (fread(m, 1, (size_t)sz, f) != (size_t)sz) { fclose(f); *err = "short read " + path; return false; }
    fclose(f);
    if (memcmp(m, "SBB1", 4) != 0 || rd32(m + 4) != 1u) { *err = "not an SBB1 v1 blob: " + path; return false; }
    uint32_t n = rd32(m + 8);
    uint64_t dir = rd64(m + 12), names = rd64(m + 20), names_len = rd64(m + 28);
    if (dir + 56ull * n > (uint64_t)sz || names + names_len > (uint64_t)sz) {
        *err = "corrupt directory in " + path;
        return false;
    }
    for (uint32_t i = 0; i < n; i++) {
        const unsigned char* r = m + dir + 56ull * i;
        uint32_t no = rd32(r);
        if (no >= names_len) { *err = "corrupt name offset in " + path; return false; }
        std::string name((const char*)(m + names + no));
        Section s;
        s.dtype = rd32(r + 4);
        uint32_t nd = rd32(r + 8);
        uint64_t cnt = 1;
        for (uint32_t d = 0; d < nd && d < 4; d++) cnt *= rd64(r + 16 + 8 * d);
        s.count = cnt;
        uint64_t off = rd64(r + 48);
        static const int esz[8] = {8, 4, 8, 4, 1, 1, 4, 1};
        if (s.dtype > 7 || off + cnt * (uint64_t)esz[s.dtype] > (uint64_t)sz) {
            *err = "section " + name + " out of range in " + path;
            return false;
        }
        s.data = m + off;
        sec_[name] = s;
    }
    return true;
}

const Section* Blob::find(const std::string& name) const {
    auto it = sec_.find(name);
    return it == sec_.end() ? nullptr : &it->second;
}

const void* Blob::typed(const std::string& name, uint32_t dt, uint64_t* count) const {
    const Section* s = find(name);
    if (!s || s->dtype != dt) { if (count) *count = 0; return nullptr; }
    if (count) *count = s->count;
    return s->data;
}

const double* Blob::f64(const std::string& n, uint64_t* c) const { return (const double*)typed(n, F64, c); }
const int64_t* Blob::i64(const std::string& n, uint64_t* c) const { return (const int64_t*)typed(n, I64, c); }
const int32_t* Blob::i32(const std::string& n, uint64_t* c) const { return (const int32_t*)typed(n, I32, c); }
const uint8_t* Blob::u8(const std::string& n, uint64_t* c) const { return (const uint8_t*)typed(n, U8, c); }

double Blob::f64_1(const std::string& name, double dflt) const {
    const double* p = f64(name);
    return p ? p[0] : dflt;
}

int64_t Blob::i64_1(const std::string& name, int64_t dflt) const {
    const int64_t* p = i64(name);
    return p ? p[0] : dflt;
}

std::string Blob::bytes(const std::string& name) const {
    const Section* s = find(name);
    if (!s) return std::string();
    static const int esz[8] = {8, 4, 8, 4, 1, 1, 4, 1};
    return std::string((const char*)s->data, (size_t)(s->count * esz[s->dtype]));
}

}  // namespace sbh
