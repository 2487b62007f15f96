// Host-side solve planner: turns one layout's system matrix and baked LU
// pattern into the level schedule the step kernel runs.
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

#include "sbb_reader.h"

namespace sbh {

// Maximum terms one lane handles in one pass (longer dot products are split
// into continuation tasks in later passes). The kernel keeps a pass's terms in
// registers, so this bounds its register arrays.
constexpr int kPlanKmax = 48;

// Per-pass record: hdr_off, word_off, nact, maxcnt, row_off, 0, 0, 0.
struct PassInfo {
    int hdr_off, word_off, nact, maxcnt, row_off, pad0, pad1, pad2;
};

struct SolvePlan {
    int n = 0, k = 0, width = 0;
    int n_slots = 0, vec_base = 0, n_levels = 0, n_tasks = 0;
    long long n_pairs = 0;           // multiply-subtract terms
    long long n_divs = 0;
    std::vector<int> pos;            // node -> permuted position
    std::vector<double> slot_init;   // [n_slots]
    std::vector<int> air_slot, air_node;   // [k]
    std::vector<PassInfo> passes;
    std::vector<int> row_off;        // per pass: maxcnt + 1 cumulative row starts
    std::vector<uint64_t> hdr;       // per active lane: target | divisor << 16 | count << 32
    std::vector<uint32_t> words;     // rows: row m of a pass holds the m-th term of every lane with count > m
    int n_pass() const { return (int)passes.size(); }
};

// Builds the plan for the factorization of A + diag(g at the coupled air
// nodes) and the two triangular solves. Fails (false, *err) when the blob is
// outside the supported model: every cell solved, symmetric permutation,
// pattern closed under elimination, one unit applied/sensed entry per column.
bool build_plan(const Blob& b, int width, SolvePlan* out, std::string* err);

}  // namespace sbh
