// Host-side solve planner: turns one layout's system matrix and baked LU
// pattern into the level schedule the step kernel runs.
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

#include "sbb_reader.h"

namespace sbh {

// Maximum terms one lane handles in one pass, and lanes one task may span (a
// segment within a 16-lane row, summed by a butterfly). Longer dot products
// are split into continuation tasks in later passes. The kernel keeps a pass's
// terms in registers, so kPlanKmax bounds its register arrays.
constexpr int kPlanKmax = 16;
constexpr int kPlanSegMax = 16;

// Per-pass record, 16 bytes: hdr_off, word_off, nact | maxcnt << 8 | has_pivot << 16 | lgmax << 17, 0.
// nact: lanes used; lgmax: log2 of the pass's widest segment (the butterfly steps it runs).
// Lane header: target | mul << 16 | inv_target << 32 | flags << 48,
// flags = log2(segment lanes) | leader << 3 | terms << 4; a lane that is not its
// segment's leader has target kSlotZero, mul kSlotOne and inv_target kSlotSink.
struct PassInfo {
    int hdr_off, word_off, packed, pad;
    int nact() const { return packed & 0xff; }
    int maxcnt() const { return (packed >> 8) & 0xff; }
    int has_pivot() const { return (packed >> 16) & 1; }
    int lgmax() const { return (packed >> 17) & 7; }
};

// Fixed slots: 0 holds 0.0 (padding terms read it), 1 is a write sink, 2 holds 1.0.
constexpr int kSlotZero = 0, kSlotSink = 1, kSlotOne = 2;
// An idle lane's header: target and reciprocal target the sink, multiplier the zero slot, not a leader.
constexpr uint64_t kIdleHeader = 0x0000000100000001ull;
// Words of padding after the last pass: a lane reads kPlanKmax words from its start.
constexpr int kWordTail = 16;
// Passes the kernel loads ahead of the one it runs plus one; the pass count is a multiple of it.
constexpr int kPlanDepth = 4;

struct SolvePlan {
    int n = 0, k = 0, width = 0;
    int n_slots = 0, vec_base = 0, inv_base = 0, n_levels = 0, n_tasks = 0;
    // term word format: 16 (a | b << 16) or 12 (a | b << 12 | v << 24, the
    // product slot[a] * slot[scale_base + v] * slot[b]); scale_base holds 1.0
    // and precedes the reciprocals (inv_base = scale_base + 1)
    int term_bits = 16, scale_base = 0;
    long long n_pairs = 0;           // multiply-subtract terms
    long long n_divs = 0;
    std::vector<int> pos;            // node -> permuted position
    std::vector<double> slot_init;   // [n_slots]
    std::vector<int> air_slot, air_node;   // [k]
    std::vector<PassInfo> passes;
    std::vector<uint64_t> hdr;       // per lane: target | mul << 16 | inv_target << 32 | flags << 48
    std::vector<uint32_t> words;     // term m of lane l at word_off + l * stride + m, stride = maxcnt rounded up to 4
                                     // (format: term_bits)
    int n_pass() const { return (int)passes.size(); }
};

// Builds the plan for the factorization of A + diag(g at the coupled air
// nodes) and the two triangular solves. Fails (false, *err) when the blob is
// outside the supported model: every cell solved, symmetric permutation,
// pattern closed under elimination, one unit applied/sensed entry per column.
bool build_plan(const Blob& b, int width, SolvePlan* out, std::string* err);

// Relaxation (Jacobi) form of the same solve, x <- D^-1 (b - O x) with
// D = diag(A) + g and O the off-diagonal part of A. It converges for every
// step when A has positive diagonal entries and
//   rho = max_i sum_{j != i} |a_ij| / a_ii < 1,
// because g >= 0 only enlarges D: rho bounds the infinity norm of the
// iteration matrix for every g, and after sweep m
//   |x* - x_m|_inf <= rho / (1 - rho) * |x_m - x_{m-1}|_inf,
// which the kernel uses as its stopping test. Row i of the device table is
// handled by lane i % 64 as its (i / 64)-th row.
constexpr int kRelaxRowsPerLane = 4;
constexpr int kRelaxRows = 64 * kRelaxRowsPerLane;   // padded row count
constexpr int kRelaxTerms = 8;                       // off-diagonal entries per row
constexpr double kRelaxRhoMax = 0.5;                 // larger bounds use the LU plan

struct RelaxPlan {
    bool ok = false;
    std::string why;                 // reason when not eligible
    int n = 0, terms = 0;            // terms: longest off-diagonal row
    double rho = 0.0;
    std::vector<double> diag;        // [kRelaxRows], padding 1.0
    std::vector<int> air_col;        // [kRelaxRows] air-side column of the node, or -1
    std::vector<double> val;         // [kRelaxTerms * kRelaxRows]: entry m of row i at m * kRelaxRows + i
    std::vector<int> col;            // same layout; padding entries are (0.0, column 0)
};

// Fills *out from the blob's A_system and the air-side columns of the LU plan
// (built first, it validates the air side). Never fails: out->ok says whether
// the relaxation form applies and out->why why not.
void build_relax(const Blob& b, const SolvePlan& lu, RelaxPlan* out);

// Block-Jacobi form: nodes grouped into blocks of at most kBlockRows (greedy,
// strongest coupling |a_ij| / min(a_ii, a_jj) first), each block solved
// exactly per sweep: x_B <- (A_BB + G_B)^-1 (b_B - A_BO x_O). When A is an
// M-matrix (off-diagonal entries <= 0, every A_BB with a non-negative inverse),
// adding g >= 0 to diagonals only shrinks |(A_BB + G_B)^-1| entrywise, so
//   rho = max_i sum_j (|A_BB^-1| |A_BO|)_ij      (at g = 0)
// bounds every step's iteration matrix in the infinity norm, with the same
// a-posteriori stopping bound as the point form. Lane l owns blocks l and
// l + 64 (block slot q = 0, 1). A block's off-block entries form one list of
// at most kBlockTerms (value, column, row within the block), so the kernel can
// fold the block inverse into them once per step and sweep with one gather per
// entry.
constexpr int kBlockRows = 3;
constexpr int kBlockSlots = 2;
constexpr int kBlockTerms = 8;                             // off-block entries per block

struct BlockPlan {
    bool ok = false;
    std::string why;
    int n_blocks = 0, terms = 0;            // terms: most off-block entries of one block
    double rho = 0.0;
    std::vector<std::vector<int>> blocks;   // node lists, ascending
    // tables, lane-minor (64 lanes), q = block slot, p / p2 = row within the block,
    // t = entry of the block's off-block list
    std::vector<int> row;                   // [(q * R + p) * 64 + lane]: node or -1
    std::vector<double> diag;               // same index: a_ii (1.0 for padding)
    std::vector<int> air;                   // same index: air column or -1
    std::vector<double> in;                 // [((q * R + p) * R + p2) * 64 + lane]: a(row p, row p2), 0 on p == p2
    std::vector<double> val;                // [(q * T + t) * 64 + lane]: entry value (0.0 padding)
    std::vector<int> col;                   // same index: its column (0 padding)
    std::vector<int> trow;                  // same index: its row within the block (0 padding)
};

void build_block(const Blob& b, const SolvePlan& lu, BlockPlan* out);

}  // namespace sbh
