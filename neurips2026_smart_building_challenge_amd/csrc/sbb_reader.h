// SBB1 scenario blob reader (host). Format as parsed by the reference loader,
// complete_port/csim/sb_baked.c:19-73: 52-byte header, 56-byte section records,
// NUL-terminated names, typed little-endian arrays.
#pragma once
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace sbh {

enum Dtype { F64 = 0, F32 = 1, I64 = 2, I32 = 3, I8 = 4, U8 = 5, U32 = 6, STR = 7 };

struct Section {
    uint32_t dtype = 0;
    uint64_t count = 0;
    const unsigned char* data = nullptr;
};

class Blob {
public:
    bool open(const std::string& path, std::string* err);
    const Section* find(const std::string& name) const;
    const double* f64(const std::string& name, uint64_t* count = nullptr) const;
    const int64_t* i64(const std::string& name, uint64_t* count = nullptr) const;
    const int32_t* i32(const std::string& name, uint64_t* count = nullptr) const;
    const uint8_t* u8(const std::string& name, uint64_t* count = nullptr) const;
    double f64_1(const std::string& name, double dflt) const;
    int64_t i64_1(const std::string& name, int64_t dflt) const;
    // raw bytes of a section (for structural hashing); empty if missing
    std::string bytes(const std::string& name) const;
    const std::string& path() const { return path_; }

private:
    const void* typed(const std::string& name, uint32_t dt, uint64_t* count) const;
    std::vector<unsigned char> buf_;
    std::map<std::string, Section> sec_;
    std::string path_;
};

}  // namespace sbh
