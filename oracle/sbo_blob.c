/* SBB1 reader for the oracle (TEST INFRASTRUCTURE).
 * Header/section layout as parsed by complete_port/csim/sb_baked.c:19-73: a
 * 52-byte header (magic, version, n_sections, dir/names offsets, names length,
 * total size, reserved) and 56-byte section records (name offset, dtype, ndim,
 * reserved, shape[4], data offset). Getters return NULL for a missing section
 * or a dtype mismatch, like sb_baked.c:91-102. The file is read into memory. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sbo.h"

static uint32_t get_u32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }
static uint64_t get_u64(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }

int sbo_blob_load(SboBlob* b, const char* path) {
    memset(b, 0, sizeof(*b));
    FILE* f = fopen(path, "rb");
    if (!f) return -1;
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (sz < 52) { fclose(f); return -1; }
    /* 64-byte aligned copy so typed views of 64-aligned data are aligned */
    b->bytes = (uint8_t*)aligned_alloc(64, ((size_t)sz + 63) / 64 * 64);
    if (!b->bytes || fread(b->bytes, 1, (size_t)sz, f) != (size_t)sz) {
        fclose(f);
        free(b->bytes);
        b->bytes = NULL;
        return -1;
    }
    fclose(f);
    b->size = (uint64_t)sz;
    const uint8_t* m = b->bytes;
    if (memcmp(m, "SBB1", 4) != 0 || get_u32(m + 4) != 1u) return -1;
    uint32_t n = get_u32(m + 8);
    uint64_t dir = get_u64(m + 12), names = get_u64(m + 20);
    b->n = (int)n;
    b->sec = (SboSec*)calloc(n ? n : 1, sizeof(SboSec));
    for (uint32_t i = 0; i < n; i++) {
        const uint8_t* r = m + dir + 56ull * i;
        SboSec* s = &b->sec[i];
        s->name = (const char*)(m + names + get_u32(r));
        s->dtype = get_u32(r + 4);
        uint32_t nd = get_u32(r + 8);
        uint64_t cnt = 1;
        for (uint32_t d = 0; d < nd && d < 4; d++) cnt *= get_u64(r + 16 + 8 * d);
        s->count = cnt;
        s->data = m + get_u64(r + 48);
    }
    return 0;
}

void sbo_blob_free(SboBlob* b) {
    free(b->sec);
    free(b->bytes);
    memset(b, 0, sizeof(*b));
}

const SboSec* sbo_sec(const SboBlob* b, const char* name) {
    for (int i = 0; i < b->n; i++)
        if (strcmp(b->sec[i].name, name) == 0) return &b->sec[i];
    return NULL;
}

static const void* typed(const SboBlob* b, const char* name, uint32_t dt) {
    const SboSec* s = sbo_sec(b, name);
    return (s && s->dtype == dt) ? s->data : NULL;
}

const double* sbo_f64(const SboBlob* b, const char* n) { return (const double*)typed(b, n, 0); }
const int64_t* sbo_i64(const SboBlob* b, const char* n) { return (const int64_t*)typed(b, n, 2); }
const int32_t* sbo_i32(const SboBlob* b, const char* n) { return (const int32_t*)typed(b, n, 3); }
const uint8_t* sbo_u8(const SboBlob* b, const char* n) { return (const uint8_t*)typed(b, n, 5); }

double sbo_f64_1(const SboBlob* b, const char* name, double dflt) {
    const double* p = sbo_f64(b, name);
    return p ? p[0] : dflt;
}

int64_t sbo_i64_1(const SboBlob* b, const char* name, int64_t dflt) {
    const int64_t* p = sbo_i64(b, name);
    return p ? p[0] : dflt;
}
