// Fused Smart Buildings env step for MI355X (gfx950).
//
// One workgroup steps a tile of up to four envs of one layout. The layout
// image and each env's state record are copied HBM -> LDS in one burst, every
// phase of the step runs out of LDS, and the record is copied back at the end.
// Each env has two wavefronts: the first runs the physics chain, the second
// (its helper) runs the work that does not feed that chain alongside it.
//
//   first wavefront
//   decode + apply     complete_port/csim/sb_sim.c:557-576, :220-244
//   HVAC pre           sb_sim.c:357-457 (lanes over VAVs / zones, wave sums)
//   field solve        sb_fdm.c:142-188 restated as (A + diag(g)) y = b: block
//                      or point relaxation with a certified stop, or numeric
//                      LU over a host-built level schedule
//   post               sb_sim.c:489-521 (boiler return, ramp)
//   observation        complete_port/csim/sb_obs.c:49-64
//   auto-reset         complete_port/pufferlib_cpu_env.h:187-208, sb_sim.c:177-218
//   helper wavefront
//   occupancy          sb_occup.c:36-61, MT19937 draws assigned by prefix sum
//                      (during decode, HVAC pre and solve: it is exogenous)
//   reward             sb_reward.c:31-155 (during the observation)
//   bookkeeping        complete_port/pufferlib_cpu_env.h:243-256
#include <hip/hip_runtime.h>

#include "sbenv.h"
#include "sbenv_internal.h"
#include "sb_philox.h"

namespace sbk {

#define RHO_AIR 1.2
#define CP_AIR 1006.0
#define RHO_W 1000.0
#define CP_W 4180.0
#define GRAV 9.8
#define PA_PER_BAR 100000.0
#define PI_D 3.14159265358979323846

enum { M_OFF = 0, M_HEAT = 1, M_COOL = 2, M_PASSIVE = 3 };

// Stamps SBK_STAMP_HELPER .. SBK_STAMP_ENTRY - 1 are the helper's.
__device__ __forceinline__ constexpr bool stamp_is_helpers(int i) {
    return i >= SBK_STAMP_HELPER && i < SBK_STAMP_ENTRY;
}

// Phase stamp of env c.e (wall clock, taken by its lane 0 when phase timing is
// on). Stamps go to the env's LDS area and are copied out by stamps_flush at
// the end of the wavefront, so taking one adds no wait on global stores.
// Stamps below SBK_STAMP_HELPER are the env's first wavefront's, the rest its helper's.
#define STAMP(i)                                                                        \
    do {                                                                                \
        if (P.phase_ts && (threadIdx.x & 63) == 0 && c.helper == stamp_is_helpers(i))     \
            c.stamps[(i)] = wall_clock64();                                             \
    } while (0)

// Orders this wavefront's LDS accesses before and after the point. A
// wavefront's LDS operations are performed in issue order, so a wavefront-scope
// fence needs no wait (nothing is emitted for it): it only keeps the compiler
// from moving memory accesses across the point, and LDS reads and writes
// still in flight stay in flight, as do global loads.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// Lane of the calling thread within its wavefront (a workgroup holds two
// wavefronts per env).
__device__ __forceinline__ int ln() { return (int)(threadIdx.x & 63); }

// Synchronisation point of one env: its wavefront's LDS writes before this
// point are visible to its LDS reads after it.
__device__ __forceinline__ void esync() { wave_lds_sync(); }

// Cross-wavefront hand-off between an env's two wavefronts (same workgroup):
// a workgroup-scope release waits for the wavefront's LDS operations
// (lgkmcnt) before the flag is written, and the waiter polls the flag, so LDS
// data written before env_post is visible to LDS reads after env_wait.
__device__ __forceinline__ void env_post(int* flag, int v) {
    esync();
    if (ln() == 0) __hip_atomic_store(flag, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void env_wait(int* flag, int v) {
    while (__builtin_amdgcn_readfirstlane(__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) < v)
        __builtin_amdgcn_s_sleep(1);
}

// Wavefront reductions and scans on DPP lane moves (no LDS traffic). Every
// lane of the wavefront must be active. The combination order is fixed:
// pairs, quads, halves of a row, rows of 16 (quad_perm, row_half_mirror,
// row_mirror), then rows 0+1 and 2+3 (row_bcast:15), then the two halves
// (row_bcast:31); lane 63 ends with the total and is broadcast.
enum {
    DPP_QUAD_1032 = 0xB1,       // quad_perm [1,0,3,2]
    DPP_QUAD_2301 = 0x4E,       // quad_perm [2,3,0,1]
    DPP_ROW_SHR = 0x110,        // + 1..15
    DPP_ROW_MIRROR = 0x140,
    DPP_ROW_HALF_MIRROR = 0x141,
    DPP_ROW_BCAST15 = 0x142,
    DPP_ROW_BCAST31 = 0x143,
};

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp_i(int old, int v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xF, false);
}

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ double dpp_d(double old, double v) {
    const unsigned long long o = __double_as_longlong(old), x = __double_as_longlong(v);
    const int lo = dpp_i<CTRL, ROWS>((int)(unsigned)o, (int)(unsigned)x);
    const int hi = dpp_i<CTRL, ROWS>((int)(unsigned)(o >> 32), (int)(unsigned)(x >> 32));
    return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}

__device__ __forceinline__ double lane63_d(double v) {
    const unsigned long long x = __double_as_longlong(v);
    const unsigned lo = __builtin_amdgcn_readlane((int)(unsigned)x, 63);
    const unsigned hi = __builtin_amdgcn_readlane((int)(unsigned)(x >> 32), 63);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

template <class Op>
__device__ __forceinline__ double wave_reduce(double v, double ident, Op op) {
    v = op(v, dpp_d<DPP_QUAD_1032>(ident, v));
    v = op(v, dpp_d<DPP_QUAD_2301>(ident, v));
    v = op(v, dpp_d<DPP_ROW_HALF_MIRROR>(ident, v));
    v = op(v, dpp_d<DPP_ROW_MIRROR>(ident, v));
    v = op(v, dpp_d<DPP_ROW_BCAST15, 0xA>(ident, v));
    v = op(v, dpp_d<DPP_ROW_BCAST31, 0xC>(ident, v));
    return lane63_d(v);
}

__device__ __forceinline__ double wave_sum(double v) {
    return wave_reduce(v, 0.0, [](double a, double b) { return a + b; });
}

__device__ __forceinline__ double wave_min(double v) {
    return wave_reduce(v, __longlong_as_double(0x7FF0000000000000ll), [](double a, double b) { return fmin(a, b); });
}

__device__ __forceinline__ double wave_max(double v) {
    return wave_reduce(v, __longlong_as_double((long long)0xFFF0000000000000ull), [](double a, double b) { return fmax(a, b); });
}

__device__ __forceinline__ int wave_isum(int v) {
    v += dpp_i<DPP_QUAD_1032>(0, v);
    v += dpp_i<DPP_QUAD_2301>(0, v);
    v += dpp_i<DPP_ROW_HALF_MIRROR>(0, v);
    v += dpp_i<DPP_ROW_MIRROR>(0, v);
    v += dpp_i<DPP_ROW_BCAST15, 0xA>(0, v);
    v += dpp_i<DPP_ROW_BCAST31, 0xC>(0, v);
    return __builtin_amdgcn_readlane(v, 63);
}

// Sum, minimum and maximum of three per-lane values in one pass (the three
// DPP chains are independent, so their latencies overlap).
__device__ __forceinline__ void wave_sum_min_max(double& s, double& mn, double& mx) {
    const double zero = 0.0, pinf = __longlong_as_double(0x7FF0000000000000ll);
    const double ninf = __longlong_as_double((long long)0xFFF0000000000000ull);
#define SBK_STEP3(CTRL, ROWS)                                 \
    s = s + dpp_d<CTRL, ROWS>(zero, s);                       \
    mn = fmin(mn, dpp_d<CTRL, ROWS>(pinf, mn));               \
    mx = fmax(mx, dpp_d<CTRL, ROWS>(ninf, mx));
    SBK_STEP3(DPP_QUAD_1032, 0xF)
    SBK_STEP3(DPP_QUAD_2301, 0xF)
    SBK_STEP3(DPP_ROW_HALF_MIRROR, 0xF)
    SBK_STEP3(DPP_ROW_MIRROR, 0xF)
    SBK_STEP3(DPP_ROW_BCAST15, 0xA)
    SBK_STEP3(DPP_ROW_BCAST31, 0xC)
#undef SBK_STEP3
    s = lane63_d(s);
    mn = lane63_d(mn);
    mx = lane63_d(mx);
}

// Sums of three per-lane values in one pass.
__device__ __forceinline__ void wave_sum3(double& a, double& b, double& d) {
#define SBK_STEP3S(CTRL, ROWS)                \
    a = a + dpp_d<CTRL, ROWS>(0.0, a);        \
    b = b + dpp_d<CTRL, ROWS>(0.0, b);        \
    d = d + dpp_d<CTRL, ROWS>(0.0, d);
    SBK_STEP3S(DPP_QUAD_1032, 0xF)
    SBK_STEP3S(DPP_QUAD_2301, 0xF)
    SBK_STEP3S(DPP_ROW_HALF_MIRROR, 0xF)
    SBK_STEP3S(DPP_ROW_MIRROR, 0xF)
    SBK_STEP3S(DPP_ROW_BCAST15, 0xA)
    SBK_STEP3S(DPP_ROW_BCAST31, 0xC)
#undef SBK_STEP3S
    a = lane63_d(a);
    b = lane63_d(b);
    d = lane63_d(d);
}

// Sums of two per-lane values in one pass.
__device__ __forceinline__ void wave_sum2(double& a, double& b) {
#define SBK_STEP2(CTRL, ROWS)                 \
    a = a + dpp_d<CTRL, ROWS>(0.0, a);        \
    b = b + dpp_d<CTRL, ROWS>(0.0, b);
    SBK_STEP2(DPP_QUAD_1032, 0xF)
    SBK_STEP2(DPP_QUAD_2301, 0xF)
    SBK_STEP2(DPP_ROW_HALF_MIRROR, 0xF)
    SBK_STEP2(DPP_ROW_MIRROR, 0xF)
    SBK_STEP2(DPP_ROW_BCAST15, 0xA)
    SBK_STEP2(DPP_ROW_BCAST31, 0xC)
#undef SBK_STEP2
    a = lane63_d(a);
    b = lane63_d(b);
}

// Sums of four per-lane values and the maximum of a fifth in one pass.
__device__ __forceinline__ void wave_sum4_max(double& a, double& b, double& d, double& e, double& mx) {
    const double ninf = __longlong_as_double((long long)0xFFF0000000000000ull);
#define SBK_STEP5(CTRL, ROWS)                               \
    a = a + dpp_d<CTRL, ROWS>(0.0, a);                      \
    b = b + dpp_d<CTRL, ROWS>(0.0, b);                      \
    d = d + dpp_d<CTRL, ROWS>(0.0, d);                      \
    e = e + dpp_d<CTRL, ROWS>(0.0, e);                      \
    mx = fmax(mx, dpp_d<CTRL, ROWS>(ninf, mx));
    SBK_STEP5(DPP_QUAD_1032, 0xF)
    SBK_STEP5(DPP_QUAD_2301, 0xF)
    SBK_STEP5(DPP_ROW_HALF_MIRROR, 0xF)
    SBK_STEP5(DPP_ROW_MIRROR, 0xF)
    SBK_STEP5(DPP_ROW_BCAST15, 0xA)
    SBK_STEP5(DPP_ROW_BCAST31, 0xC)
#undef SBK_STEP5
    a = lane63_d(a);
    b = lane63_d(b);
    d = lane63_d(d);
    e = lane63_d(e);
    mx = lane63_d(mx);
}

// Per-AHU sums by one lane each: lane a (< na) adds vals[t] over its list
// positions t in [off[a], off[a + 1]) in order. The per-AHU terms were written
// at their entry's position in the AHU's list (ascending VAVs or columns: the
// order csim accumulates them in), so an AHU's terms are contiguous and a
// batch of eight loads goes out before its adds; with COUNT also the number of
// terms > 0. The terms are non-negative (flows, temperatures in K times
// areas). The calling wavefront wrote them before an esync().
template <bool COUNT>
__device__ __forceinline__ double ahu_range_sum(const double* vals, const int* off, int a, int& npos) {
    double s = 0.0;
    int np = 0;
    const int t1 = off[a + 1];
    for (int t = off[a]; t < t1; t += 8) {
        // past the list's end the loads repeat its last term and the adds take
        // +0.0, which leaves the (non-negative) sum unchanged
        double v8[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v8[u] = vals[min(t + u, t1 - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const double x = t + u < t1 ? v8[u] : 0.0;
            s += x;
            if (COUNT) np += x > 0.0 ? 1 : 0;
        }
    }
    npos = np;
    return s;
}

// Per-AHU sums of the list-ordered terms: lane a (< na) receives AHU a's. A
// single AHU (a layout's whole VAV or column list, 40-128 terms) is summed over
// the whole wavefront (one load a lane, a DPP tree); with more AHUs (fewer
// terms each) one lane per AHU adds its terms in list order (ahu_range_sum).
// Every lane of the wavefront must call it.
template <bool COUNT>
__device__ __forceinline__ double ahu_sums_of(const double* vals, const int* off, int na, int& npos) {
    double sv = 0.0;
    int np = 0;
    if (na == 1) {
        const int t1 = off[1];
        int k = 0;
        for (int t = ln(); t < t1; t += 64) {
            const double v = vals[t];
            sv += v;
            if (COUNT) k += v > 0.0 ? 1 : 0;
        }
        sv = wave_sum(sv);
        if (COUNT) np = wave_isum(k);
    } else if (ln() < na) {
        sv = ahu_range_sum<COUNT>(vals, off, ln(), np);
    }
    npos = np;
    return sv;
}

// Inclusive prefix sum over the wavefront.
__device__ __forceinline__ int wave_iscan(int v) {
    v += dpp_i<DPP_ROW_SHR + 1>(0, v);
    v += dpp_i<DPP_ROW_SHR + 2>(0, v);
    v += dpp_i<DPP_ROW_SHR + 4>(0, v);
    v += dpp_i<DPP_ROW_SHR + 8>(0, v);
    v += dpp_i<DPP_ROW_BCAST15, 0xA>(0, v);
    v += dpp_i<DPP_ROW_BCAST31, 0xC>(0, v);
    return v;
}

// Env-wide reductions (one wavefront per env); every lane receives the value.
template <int W>
__device__ __forceinline__ double bsum(double v, double*) { return wave_sum(v); }

template <int W>
__device__ __forceinline__ double bmin(double v, double*) { return wave_min(v); }

template <int W>
__device__ __forceinline__ double bmax(double v, double*) { return wave_max(v); }

template <int W>
__device__ __forceinline__ int bisum(int v, double*) { return wave_isum(v); }

// Exclusive prefix sum of an int per lane over the env's wavefront; *total
// receives the sum.
template <int W>
__device__ __forceinline__ int bscan(int v, int*, int* total) {
    const int inc = wave_iscan(v);
    *total = __builtin_amdgcn_readlane(inc, 63);
    return inc - v;
}

// Layout tables in the staged LDS image (shared by the envs of a workgroup):
// each accessor adds the table's offset (constant memory, kept in the scalar
// cache) to the image base, so no table pointer has to stay live in registers.
struct Tab {
    const unsigned char* img;
    const SBK_C ImgLayout* g;
#define SBK_TAB(T, name) \
    __device__ __forceinline__ const T* name() const { return reinterpret_cast<const T*>(img + g->name); }
    SBK_TAB(double, cap)
    SBK_TAB(double, mcoup)
    SBK_TAB(double, mret)
    SBK_TAB(double, mgain)
    SBK_TAB(double, solar_c)
    SBK_TAB(double, rx_diag)
    SBK_TAB(double, zone_area)
    SBK_TAB(double, vav_area)
    SBK_TAB(double, vav_c)
    SBK_TAB(double, ahu_c)
    SBK_TAB(double, act_mn)
    SBK_TAB(double, act_mx)
    SBK_TAB(double, act_mnr)
    SBK_TAB(double, act_mxr)
    SBK_TAB(double, act_hi)
    SBK_TAB(double, f_mean)
    SBK_TAB(double, f_sd)
    SBK_TAB(int, rx_air)
    SBK_TAB(int, pos)
    SBK_TAB(int, zone_cell_off)
    SBK_TAB(int, zone_cells)
    SBK_TAB(int, vz_off)
    SBK_TAB(int, vz_idx)
    SBK_TAB(int, vav_ahu)
    SBK_TAB(int, coupled)
    SBK_TAB(int, zone_col_off)
    SBK_TAB(int, zone_cols)
    SBK_TAB(int, act_src)
    SBK_TAB(int, air_slot)
    SBK_TAB(int, air_node)
    SBK_TAB(int, ahu_vav_off)
    SBK_TAB(int, ahu_vavs)
    SBK_TAB(int, ahu_col_off)
    SBK_TAB(int, ahu_cols)
    SBK_TAB(int, vav_lpos)
    SBK_TAB(int, col_lpos)
    SBK_TAB(double, ahu_area)
    SBK_TAB(int, cv_off)
    SBK_TAB(int, cv_node)
    SBK_TAB(int, cv_coff)
    SBK_TAB(int, cv_cidx)
    SBK_TAB(uint32_t, f_src)
    SBK_TAB(uint32_t, act_dst)
    SBK_TAB(uint32_t, act_aux)
    SBK_TAB(uint8_t, is_room)
    SBK_TAB(uint8_t, act_disc)
    SBK_TAB(uint8_t, act_flags)
#undef SBK_TAB
};

struct Ctx {
    const SBK_C DevLayout* L;
    const SBK_C DevScen* S;
    int e;                   // env index
    bool helper;             // the env's second wavefront
    bool conv;               // stochastic convection on (read with the env's records, before the burst)
    unsigned long long* stamps;   // phase stamps (LDS)
    unsigned char* rec;      // HBM record of this env
    Tab t;
    double *T, *M, *damper, *reheat, *ratio, *heatsp, *coolsp, *dcmd, *rcmd, *sensing;
    double *recirc, *sat, *fan, *flow, *plant;
    int *run, *coolreq, *ip;
    uint8_t *mode, *prev_valid, *dcmd_set, *rcmd_set, *occ_state, *occV;
    double *slots, *zq, *unres, *fdem, *rwen, *lsum, *g, *tair;
    double *wsum, *atotal, *satv, *demand, *fdsum, *red, *misc;
    double* cal;             // the two calendar sections of the state image
    const double* row;       // this step's calendar values (RW_*), the aux-time row after them
    uint32_t* mt;
    int* iscr;
    unsigned char* prec;     // LDS copy of the solve pass records
    const float* act;        // the step's action row (LDS)
    const unsigned char* imgb;   // layout image (LDS)
    unsigned char* envb;         // this env's LDS region
    double* obsx;                // per-step values the observation reads (OX_*)
    const double *dirx, *elec_wk, *elec_we, *elec_co2, *gas_price;   // scenario image (LDS)
};

// img: the workgroup's layout image; env: this env's LDS region.
__device__ __forceinline__ void bind(Ctx& c, const unsigned char* img, unsigned char* env) {
    const SBK_C DevLayout* L = c.L;
    c.t.img = img;
    c.t.g = &L->img;
    c.imgb = img;
    c.envb = env;
    c.obsx = (double*)(env + L->lds.obsx);
    const LdsLayout l = L->lds;
    unsigned char* s = env + l.state;
    const StateLayout st = L->st;
    c.T = (double*)(s + st.T);
    c.M = (double*)(s + st.M);
    c.damper = (double*)(s + st.damper);
    c.reheat = (double*)(s + st.reheat);
    c.ratio = (double*)(s + st.ratio);
    c.heatsp = (double*)(s + st.heatsp);
    c.coolsp = (double*)(s + st.coolsp);
    c.dcmd = (double*)(s + st.dcmd);
    c.rcmd = (double*)(s + st.rcmd);
    c.sensing = (double*)(s + st.sensing);
    c.recirc = (double*)(s + st.recirc);
    c.sat = (double*)(s + st.sat);
    c.fan = (double*)(s + st.fan);
    c.flow = (double*)(s + st.flow);
    c.plant = (double*)(s + st.plant);
    c.cal = (double*)(s + st.cal);
    c.run = (int*)(s + st.run);
    c.coolreq = (int*)(s + st.coolreq);
    c.ip = (int*)(s + st.iplant);
    c.mode = s + st.mode;
    c.prev_valid = s + st.prev_valid;
    c.dcmd_set = s + st.dcmd_set;
    c.rcmd_set = s + st.rcmd_set;
    c.occ_state = s + st.occ_state;
    c.occV = s + st.occV;
    c.mt = (uint32_t*)(env + l.mt);
    const ScenImg si = c.S->img;
    const unsigned char* sc = env + l.scen;
    c.dirx = (const double*)(sc + si.dirx);
    c.elec_wk = (const double*)(sc + si.elec_wk);
    c.elec_we = (const double*)(sc + si.elec_we);
    c.elec_co2 = (const double*)(sc + si.elec_co2);
    c.gas_price = (const double*)(sc + si.gas_price);
    c.act = (const float*)(env + l.act);
    c.slots = (double*)(env + l.slots);
    c.zq = (double*)(env + l.zq);
    c.unres = (double*)(env + l.vtmp);
    c.fdem = c.unres + L->nv;
    c.rwen = c.fdem + L->nv;
    c.lsum = c.rwen + L->nv;
    c.g = (double*)(env + l.g);
    c.tair = (double*)(env + l.tair);
    double* a = (double*)(env + l.atmp);
    c.wsum = a;
    c.atotal = a + L->na;
    c.satv = a + 2 * L->na;
    c.demand = a + 3 * L->na;
    c.fdsum = a + 4 * L->na;
    c.red = (double*)(env + l.red);
    c.misc = (double*)(env + l.misc);
    c.iscr = (int*)(env + l.iscr);
    c.prec = env + l.prec;
}

// ------------------------------------------------------------------ helpers
__device__ __forceinline__ double ahu_static(const Ctx& c, int a) {
    if (c.run[a] != 1) return 0.0;
    double sp = c.fan[a], mn = c.t.ahu_c()[a * 9 + 2];
    return sp > mn ? sp : mn;
}

__device__ __forceinline__ double vav_unrestricted(const Ctx& c, int v) {
    const double* vc = c.t.vav_c() + v * 9;
    double d = c.damper[v] * vc[0] * sqrt(ahu_static(c, c.t.vav_ahu()[v]) / vc[4]);
    return d > 0.00001 ? d : 0.00001;
}

__device__ __forceinline__ double total_flow_rate(const Ctx& c) {
    double ff = c.misc[MS_FFS];
    double dp = (c.ip[PI_PUMP_RUN] != 1) ? 0.0 : GRAV * RHO_W * c.plant[PF_PUMP_HEAD] / PA_PER_BAR;
    return ff * sqrt(dp / (1.0 + ff * ff * c.S->header_res)) / 3600.0;
}

__device__ __forceinline__ int default_mode(int cur, double zt, double hsp, double csp) {
    double mid = 0.5 * (csp - hsp) + hsp;
    if (zt < hsp) return M_HEAT;
    if (zt > csp) return M_COOL;
    if (zt < mid && cur == M_HEAT) return M_HEAT;
    if (zt > mid && cur == M_COOL) return M_COOL;
    return M_OFF;
}

// Passes of a U-slot loop: U = 1 serves counts up to 64 (one pass), U = 2
// counts up to 64 * SBK_VPL (the callers dispatch on the count).
template <int U>
__device__ constexpr int upasses() { return U == 1 ? 1 : SBK_VPL / U; }

// zone means of room cells (ascending), sb_sim.c:149-160. U zones per lane
// per pass (lane + 64 u) with their cell chains interleaved.
template <int U>
__device__ __forceinline__ void zone_means_pass(Ctx& c, double* out) {
    const int nz = c.L->nz, lane = ln();
#pragma unroll
    for (int pass = 0; pass < upasses<U>(); pass++) {
        const int base = pass * 64 * U;
        if (base >= nz) break;
        int z[U], a[U], b[U];
        bool ok[U];
        double sum[U];
        int len = 0;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int zz = base + 64 * u + lane;
            ok[u] = zz < nz;
            z[u] = ok[u] ? zz : nz - 1;
            a[u] = c.t.zone_cell_off()[z[u]];
            b[u] = c.t.zone_cell_off()[z[u] + 1];
            sum[u] = 0.0;
            len = max(len, b[u] - a[u]);
        }
        for (int i = 0; i < len; i++) {
            double tv[U];
#pragma unroll
            for (int u = 0; u < U; u++) tv[u] = c.T[c.t.zone_cells()[a[u] + i < b[u] ? a[u] + i : a[u]]];
#pragma unroll
            for (int u = 0; u < U; u++)
                if (a[u] + i < b[u]) sum[u] += tv[u];
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (ok[u]) out[z[u]] = sum[u] / (double)(b[u] - a[u]);
    }
}

template <int W>
__device__ __forceinline__ void zone_means(Ctx& c, double* out) {
    if (c.L->nz > 64) zone_means_pass<2>(c, out);
    else zone_means_pass<1>(c, out);
}

// area-weighted VAV temperatures from zone means (sb_sim.c:163-175) of the U
// VAVs v[u], their zone chains interleaved (each VAV's zones in order)
template <int U>
__device__ __forceinline__ void vav_temps(const Ctx& c, const double* zmean, const int (&v)[U], double (&tv)[U],
                                          double (&area)[U]) {
    int a[U], b[U];
    double wt[U];
    int len = 0;
#pragma unroll
    for (int u = 0; u < U; u++) {
        a[u] = c.t.vz_off()[v[u]];
        b[u] = c.t.vz_off()[v[u] + 1];
        area[u] = 0.0;
        wt[u] = 0.0;
        len = max(len, b[u] - a[u]);
    }
    for (int i = 0; i < len; i++) {
        double za[U], zm[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int z = c.t.vz_idx()[a[u] + i < b[u] ? a[u] + i : a[u]];
            za[u] = c.t.zone_area()[z];
            zm[u] = zmean[z];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (a[u] + i < b[u]) {
                area[u] += za[u];
                wt[u] += zm[u] * za[u];
            }
        }
    }
#pragma unroll
    for (int u = 0; u < U; u++) tv[u] = (area[u] > 0.0) ? wt[u] / area[u] : 0.0;
}

// area-weighted VAV temperature from zone means (sb_sim.c:163-175)
__device__ __forceinline__ double vav_temp(const Ctx& c, const double* zmean, int v, double* area_out) {
    const SBK_C DevLayout* L = c.L;
    double area = 0.0, wt = 0.0;
    for (int t = c.t.vz_off()[v]; t < c.t.vz_off()[v + 1]; t++) {
        int z = c.t.vz_idx()[t];
        area += c.t.zone_area()[z];
        wt += zmean[z] * c.t.zone_area()[z];
    }
    *area_out = area;
    return (area > 0.0) ? wt / area : 0.0;
}

// ------------------------------------------------------------------ observation
// Values the observation reads besides the state (sb_obs.c:49-64 device
// fields): per AHU the static pressure, delivered flow, flow fraction and
// outside-air flow; the pump differential pressure; the row's ambient.
// VAV sensed temperatures of the step (area-weighted zone means of the field
// before the step, sb_sim.c:368-377), computed by the helper wavefront for
// the first wavefront's VAV pass: the temperature goes to c.sensing, and
// c.fdem (scratch until the coupled-column pass) holds the VAV's zone area,
// whose sign says whether the VAV senses a zone at all.
// The VAVs' terms of their AHU's return-air mean: sensing * area into c.rwen
// at the VAV's position in its AHU's list (the coupled-column pass writes
// c.rwen only after the first wavefront has waited for these sums); the
// areas' per-AHU sums are a layout table (every VAV has zone area: the host
// refuses one without).
template <int U>
__device__ __forceinline__ void vav_sensing(Ctx& c) {
    const int nv = c.L->nv, lane = ln();
#pragma unroll
    for (int pass = 0; pass < upasses<U>(); pass++) {
        const int base = pass * 64 * U;
        if (base >= nv) break;
        int v[U];
        bool ok[U];
        double tv[U], area[U], varea[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int vv0 = base + 64 * u + lane;
            ok[u] = vv0 < nv;
            v[u] = ok[u] ? vv0 : nv - 1;
            varea[u] = c.t.vav_area()[v[u]];
        }
        vav_temps<U>(c, c.zq, v, tv, area);
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (ok[u]) {
                c.sensing[v[u]] = tv[u];
                c.fdem[v[u]] = area[u];
                c.rwen[c.t.vav_lpos()[v[u]]] = tv[u] * varea[u];
            }
        }
    }
}

template <int W>
__device__ __forceinline__ void obs_specials(Ctx& c, double amb) {
#pragma clang fp contract(off)
    const int l = ln();
    double* ox = c.obsx;
    if (l < c.L->na) {
        const int a = l;
        double* ax = ox + OX_AHU + 4 * a;
        ax[0] = ahu_static(c, a);
        ax[1] = (c.run[a] == 1) ? c.flow[a] : 0.0;
        ax[2] = c.flow[a] / c.t.ahu_c()[a * 9 + 1];
        ax[3] = (1.0 - c.recirc[a]) * c.flow[a];
    }
    if (l == 0) {
        ox[OX_AMB] = amb;
        ox[OX_DP] = (c.ip[PI_PUMP_RUN] == 1) ? 9.8 * 1000.0 * c.plant[PF_PUMP_HEAD] / 100000.0 : 0.0;
    }
    esync();
}

// Observation row (sb_obs.c:49-64) at a calendar row whose ambient is `amb`
// and aux-time values `aux` (n_aux - 1). Every device field is a gather from
// its host-resolved source, normalised as (f32(v) - mean) / sd; fields are
// taken four per lane at a time so their LDS reads overlap.
template <int W>
__device__ __forceinline__ void write_obs(Ctx& c, float* row, double amb, const double* aux, bool tail) {
#pragma clang fp contract(off)
    obs_specials<W>(c, amb);
    const SBK_C DevLayout* L = c.L;
    const int nd = L->n_dev;
    constexpr int U = 4;
    for (int i0 = 0; i0 < nd; i0 += U * W) {
        uint32_t src[U];
        double mean[U], sd[U], v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * W + ln();
            const int ic = i < nd ? i : nd - 1;
            src[u] = c.t.f_src()[ic];
            mean[u] = c.t.f_mean()[ic];
            sd[u] = c.t.f_sd()[ic];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const unsigned char* base = (src[u] & OBS_SRC_IMG) ? c.imgb : c.envb;
            const unsigned char* p = base + (src[u] & OBS_SRC_OFF);
            v[u] = (src[u] & OBS_SRC_I32) ? (double)*reinterpret_cast<const int*>(p)
                                          : *reinterpret_cast<const double*>(p);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (i0 + u * W >= nd) break;   // wave-uniform: slots past the field count
            const int i = i0 + u * W + ln();
            const float v32 = (float)v[u];
            if (i < nd) __builtin_nontemporal_store((float)((sd[u] > 0.0) ? ((double)v32 - mean[u]) / sd[u] : 0.0), row + i);
        }
    }
    const int na = L->n_aux;
    for (int i = ln(); i < na - 1; i += W) row[L->n_dev + i] = (float)aux[i];
    int occ = 0;
    for (int z = ln(); z < L->nz; z += W) occ += c.occV[z];
    occ = bisum<W>(occ, c.red);
    if (ln() == 0) row[L->n_dev + na - 1] = (float)occ;
    // the row's padding past the observation is zeroed by puf_reset only: no
    // step writes there afterwards (the reference GPU env writes obs_len floats)
    if (tail)
        for (int i = L->n_dev + na + ln(); i < 1024; i += W) __builtin_nontemporal_store(0.0f, row + i);
}

// ------------------------------------------------------------------ occupancy
__device__ __forceinline__ uint32_t mt_temper(uint32_t y) {
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

__device__ __forceinline__ uint32_t mt_mix(uint32_t cur, uint32_t nxt, uint32_t far) {
    uint32_t x = (cur & 0x80000000u) | (nxt & 0x7fffffffu);
    uint32_t xa = x >> 1;
    if (x & 1u) xa ^= 0x9908b0dfu;
    return far ^ xa;
}

// MT19937 twist of the 624-word state in LDS, in three dependency phases:
// words [0,227) read only old words, [227,454) read phase-1 words at i-227,
// [454,624) read phase-2 words (and word 623 reads the new word 0).
template <int W>
__device__ __forceinline__ void mt_twist(uint32_t* mt) {
    constexpr int PER = (227 + W - 1) / W;
    uint32_t v[PER];
#pragma unroll
    for (int ph = 0; ph < 3; ph++) {
        const int lo = ph * 227, hi = ph == 2 ? 624 : lo + 227;
#pragma unroll
        for (int r = 0; r < PER; r++) {
            int i = lo + ln() + r * W;
            if (i < hi) {
                uint32_t nxt = (i == 623) ? mt[0] : mt[i + 1];
                uint32_t far = (ph == 0) ? mt[i + 397] : mt[i - 227];
                v[r] = mt_mix(mt[i], nxt, far);
            }
        }
        esync();
#pragma unroll
        for (int r = 0; r < PER; r++) {
            int i = lo + ln() + r * W;
            if (i < hi) mt[i] = v[r];
        }
        esync();
    }
}

// Tempered words at stream positions idx + 2d, idx + 2d + 1 (below 624) for
// each drawing occupant of this lane; d counts draws from `first`.
template <int MAXC, class Ptr>
__device__ __forceinline__ void gather_words(Ptr src, int idx, int first, const int* need, uint32_t* w) {
    int d = first;
#pragma unroll
    for (int r = 0; r < MAXC; r++) {
        w[2 * r] = 0;
        w[2 * r + 1] = 0;
        if (need[r]) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int pos = idx + 2 * d + h;
                if (pos < SBK_MT_N) w[2 * r + h] = mt_temper(src[pos]);
            }
            d++;
        }
    }
}

// One interval of the RandomizedArrivalDeparture chains (sb_occup.c:36-61).
// Occupant o = z * nassign + a draws iff it is at home in the arrival window
// or at work in the departure window of a workday; draws are taken from the
// MT stream in occupant order, so occupant o uses the words at
// 2 * (number of drawing occupants before o). The new chain states go to
// st_out (which may be c.occ_state itself) and the zone counts to v_out.
// Returns whether the draws twisted the state (staged through c.mt).
template <int W>
__device__ __forceinline__ bool occupancy_advance(Ctx& c, int hour, int workday, uint8_t* st_out, uint8_t* v_out) {
    const SBK_C DevLayout* L = c.L;
    const SBK_C DevScen* S = c.S;
    const int nocc = L->nz * L->nassign;
    constexpr int MAXC = 5;   // occupants per lane (nocc <= 5 * W, checked on the host)
    const int per = (nocc + W - 1) / W;
    const int o0 = ln() * per;
    int need[MAXC];
    int cnt = 0;
#pragma unroll
    for (int r = 0; r < MAXC; r++) {
        need[r] = 0;
        int o = o0 + r;
        if (r < per && o < nocc && workday) {
            int st = c.occ_state[o];
            if (st == 0) need[r] = (hour >= S->ea && hour <= S->la);
            else need[r] = (hour >= S->ed && hour < S->ld);
        }
        cnt += need[r];
    }
    int total;
    int first = bscan<W>(cnt, c.iscr, &total);
    const int idx = c.ip[PI_MT_IDX];
    const int words = 2 * total;
    uint32_t* hbm_mt = (uint32_t*)(c.rec + L->st.mt);
    // the draws need the rest of the current block and the start of the next
    const bool twisted = total > 0 && idx + words > SBK_MT_N;
    // gather the tempered words: stream position s -> old[idx + s] or new[idx + s - 624];
    // words before the twist are read from the old state in HBM (the state is
    // not staged: most steps draw nothing), the rest after a twist in LDS
    uint32_t w_old[2 * MAXC];
#pragma unroll
    for (int r = 0; r < 2 * MAXC; r++) w_old[r] = 0;
    if (total > 0) gather_words<MAXC>(hbm_mt, idx, first, need, w_old);
    if (twisted) {
        for (int i = ln(); i < SBK_MT_N; i += W) c.mt[i] = hbm_mt[i];
        esync();
        mt_twist<W>(c.mt);
        int d = first;
#pragma unroll
        for (int r = 0; r < MAXC; r++) {
            if (need[r]) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    int pos = idx + 2 * d + h;
                    if (pos >= SBK_MT_N) w_old[2 * r + h] = mt_temper(c.mt[pos - SBK_MT_N]);
                }
                d++;
            }
        }
        for (int i = ln(); i < SBK_MT_N; i += W) hbm_mt[i] = c.mt[i];
        // the only reader of these words within this kernel is this env's
        // reset path (the reset's second interval), on a wavefront of this
        // workgroup, after a hand-off or in program order: a workgroup-scope
        // fence orders it (an agent-scope one would write back and invalidate
        // the whole L2 of the XCD); later launches see the words across the
        // kernel boundary
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    }
    // apply the chain updates
#pragma unroll
    for (int r = 0; r < MAXC; r++) {
        int o = o0 + r;
        if (r < per && o < nocc) {
            int st = c.occ_state[o];
            if (!workday) {
                st = 0;
            } else if (st == 0) {
                if (need[r]) {
                    double u = ((w_old[2 * r] >> 5) * 67108864.0 + (w_old[2 * r + 1] >> 6)) / 9007199254740992.0;
                    if (u < S->p_arr) st = 1;
                }
            } else if (hour < S->ed) {
            } else if (hour >= S->ld) {
                st = 0;
            } else if (need[r]) {
                double u = ((w_old[2 * r] >> 5) * 67108864.0 + (w_old[2 * r + 1] >> 6)) / 9007199254740992.0;
                if (u < S->p_dep) st = 0;
            }
            st_out[o] = (uint8_t)st;
        }
    }
    esync();
    if (ln() == 0 && total > 0) {
        int ni = idx + words;
        c.ip[PI_MT_IDX] = twisted ? ni - SBK_MT_N : ni;
    }
    for (int z = ln(); z < L->nz; z += W) {
        int s = 0;
        for (int a = 0; a < L->nassign; a++) s += st_out[z * L->nassign + a];
        v_out[z] = (uint8_t)s;
    }
    esync();
    return twisted;
}

// ------------------------------------------------------------------ convection
// Stochastic convection (complete_port/csim/sb_convect.c:39-73) splits into a
// plan and an apply. Which cells swap depends only on the convection stream,
// never on temperatures, so the helper wavefront draws the step's swaps while
// the first wavefront runs the HVAC pre-step and the solve, and hands over the
// permutation they compose to; the first wavefront applies it to the new
// field after the solve (sb_sim.c:489).
//
// Stream words come from a window of SBK_CV_WIN tempered words in LDS at
// stream positions [wb, wb + SBK_CV_WIN); positions count from the start of
// the state block in c.mt (the env's state, staged from HBM), and a fill that
// runs past the block's end twists the state and rebases every position by
// -624. A round reads ahead of what it consumes, so the step may end before
// the first word of a block it twisted into (a negative position): the HBM
// state then stays the block before (twisting writes that block to HBM first
// when it is not the one staged).
struct CvStream {
    uint32_t* win;
    uint32_t* hbm;   // the env's stream state in its HBM record
    int wb, pos;
    bool twisted;
};

// Refills the window to start at s.pos: words still in the old window are
// kept, the rest tempered from the state (twisting it when they run past the
// block's end).
template <int W>
__device__ __forceinline__ void cv_fill(CvStream& s, uint32_t* mt) {
    constexpr int PER = SBK_CV_WIN / W;
    uint32_t v[PER];
    const int old_end = s.wb + SBK_CV_WIN;
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int q = s.pos + ln() + r * W;
        v[r] = 0u;
        if (q < old_end) v[r] = s.win[q - s.wb];
        else if (q < SBK_MT_N) v[r] = mt_temper(mt[q]);
    }
    const bool tw = s.pos + SBK_CV_WIN > SBK_MT_N;
    if (tw) {
        if (s.twisted)
            for (int i = ln(); i < SBK_MT_N; i += W) s.hbm[i] = mt[i];
        esync();
        mt_twist<W>(mt);
#pragma unroll
        for (int r = 0; r < PER; r++) {
            const int q = s.pos + ln() + r * W;
            if (q >= SBK_MT_N && q >= old_end) v[r] = mt_temper(mt[q - SBK_MT_N]);
        }
    }
    esync();
#pragma unroll
    for (int r = 0; r < PER; r++) s.win[ln() + r * W] = v[r];
    esync();
    s.wb = s.pos;
    if (tw) {
        s.wb -= SBK_MT_N;
        s.pos -= SBK_MT_N;
        s.twisted = true;
    }
}

// Next stream word (wave-uniform).
template <int W>
__device__ __forceinline__ uint32_t cv_next(CvStream& s, uint32_t* mt) {
    if (s.pos >= s.wb + SBK_CV_WIN) cv_fill<W>(s, mt);
    return __builtin_amdgcn_readfirstlane(s.win[s.pos++ - s.wb]);
}

// Uniform integer in [0, max] by masked rejection (sb_rng.c:45-54).
template <int W>
__device__ __forceinline__ int cv_interval(CvStream& s, uint32_t* mt, uint32_t max) {
    if (max == 0u) return 0;
    uint32_t mask = max;
    mask |= mask >> 1;
    mask |= mask >> 2;
    mask |= mask >> 4;
    mask |= mask >> 8;
    mask |= mask >> 16;
    uint32_t v;
    do {
        v = cv_next<W>(s, mt) & mask;
    } while (v > max);
    return (int)v;
}

// The helper's half: draws the step's swaps in the stream order of
// sb_conv_apply and composes them into the permutation sig of the room
// cells (the new field at cell s is the old field at cell sig[s]). The stream
// state arrives in c.mt with the staging burst; `restage` reloads it from HBM
// (the occupancy draws of this step twisted their own state through c.mt).
// A round reads the u of up to 64 undecided cells in parallel, each at the
// position it has if no cell before it swaps; the first cell that swaps fixes
// where the stream continues.
template <int W>
__device__ __forceinline__ void conv_plan(Ctx& c, bool restage) {
    const SBK_C DevLayout* L = c.L;
    const double p = c.S->conv_p;
    uint32_t* mt = c.mt;
    const uint32_t* hbm_mt = reinterpret_cast<const uint32_t*>(c.rec + L->st.cmt);
    int* sig = reinterpret_cast<int*>(c.envb + L->lds.cvsig);
    int* lft = reinterpret_cast<int*>(c.envb + L->lds.cvl);
    int* rgt = reinterpret_cast<int*>(c.envb + L->lds.cvr);
    const int* off = c.t.cv_off();
    const int* coff = c.t.cv_coff();
    const int* cidx = c.t.cv_cidx();
    if (restage)
        for (int i = ln(); i < SBK_MT_N; i += W) mt[i] = hbm_mt[i];
    for (int i = ln(); i < L->cv_cells; i += W) sig[i] = i;
    esync();
    CvStream s;
    s.win = reinterpret_cast<uint32_t*>(c.envb + L->lds.cvwin);
    s.hbm = reinterpret_cast<uint32_t*>(c.rec + L->st.cmt);
    s.pos = c.ip[PI_CONV_IDX];
    s.wb = s.pos - SBK_CV_WIN;   // empty window
    s.twisted = false;
    cv_fill<W>(s, mt);
    // rounds over the cells in stream order, across rooms while the current
    // room holds no pair yet (a room's end then draws nothing), else up to its
    // end (where its pairs are shuffled). Room ends (lane r: the end of room r)
    // and which cells have candidates (bit c % 64 of word c / 64) stay in
    // registers, so a round's only LDS reads are its stream words.
    const int ncells = L->cv_cells, nrooms = L->cv_rooms;
    const int rend_l = ln() < nrooms ? off[ln() + 1] : 0x7fffffff;
    uint64_t hasc[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int cg = ln() + W * r;
        hasc[r] = __ballot(cg < ncells && coff[cg + 1] > coff[cg]);
    }
    // the room holding cell x (rooms are consecutive; empty ones hold none)
    auto room_of = [&](int x) { return __popcll(__ballot(rend_l <= x)); };
    int g = 0, m = 0;
    while (g < ncells) {
        const int room = room_of(g);
        const int rend = __builtin_amdgcn_readlane(rend_l, room);
        const int h = min(m == 0 ? ncells : rend, g + W);
        if (s.pos + 2 * (h - g) > s.wb + SBK_CV_WIN) cv_fill<W>(s, mt);
        const int i = ln();
        bool sel = false;
        if (i < h - g) {
            const uint32_t a = s.win[s.pos - s.wb + 2 * i], b = s.win[s.pos - s.wb + 2 * i + 1];
            const double u = ((a >> 5) * 67108864.0 + (b >> 6)) / 9007199254740992.0;
            const int cg = g + i, q = cg >> 6;
            const uint64_t hw = q == 0 ? hasc[0] : (q == 1 ? hasc[1] : (q == 2 ? hasc[2] : hasc[3]));
            sel = !(u > p) && ((hw >> (cg & 63)) & 1ull);
        }
        const uint64_t bal = __ballot(sel);
        bool close = false;   // the current room's pairs are complete after this round
        if (bal == 0ull) {
            s.pos += 2 * (h - g);
            close = rend <= h;
            g = h;
        } else {
            const int first = __builtin_ctzll(bal);
            const int gs = g + first;
            s.pos += 2 * (first + 1);
            const int grend = __builtin_amdgcn_readlane(rend_l, room_of(gs));   // rooms passed held no pair
            const int c0 = coff[gs], c1 = coff[gs + 1];
            const int pick = cv_interval<W>(s, mt, (uint32_t)(c1 - c0 - 1));
            if (ln() == 0) {
                lft[m] = gs;
                rgt[m] = cidx[c0 + pick];
            }
            m++;
            g = gs + 1;
            close = g == grend;
        }
        if (close && m > 0) {
            // Fisher-Yates over the room's pairs, last first (sb_convect.c:60-64),
            // then the swaps in order composed into sig (:65-71)
            for (int t = m - 1; t > 0; t--) {
                const int j2 = cv_interval<W>(s, mt, (uint32_t)t);
                if (ln() == 0) {
                    const int l0 = lft[t], r0 = rgt[t];
                    lft[t] = lft[j2];
                    rgt[t] = rgt[j2];
                    lft[j2] = l0;
                    rgt[j2] = r0;
                }
            }
            if (ln() == 0) {
                for (int t = 0; t < m; t++) {
                    const int a = lft[t], b = rgt[t];
                    const int x = sig[a];
                    sig[a] = sig[b];
                    sig[b] = x;
                }
            }
            m = 0;
        }
    }
    esync();
    // the state of the block holding the next unread position: the twisted
    // one, or (a negative position) the block before, already in HBM
    if (s.twisted && s.pos >= 0)
        for (int i = ln(); i < SBK_MT_N; i += W) s.hbm[i] = mt[i];
    // read again only by later launches (across the kernel boundary)
    if (s.twisted) __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    if (ln() == 0) c.ip[PI_CONV_IDX] = s.pos < 0 ? s.pos + SBK_MT_N : s.pos;
    esync();
}

// The first wavefront's half: the new field of room cell s is the field at
// cell sig[s] after the solve.
template <int W>
__device__ __forceinline__ void conv_apply(Ctx& c) {
    const SBK_C DevLayout* L = c.L;
    const int* node = c.t.cv_node();
    const int* sig = reinterpret_cast<const int*>(c.envb + L->lds.cvsig);
    constexpr int PER = 4;   // room cells per lane (at most 256, checked on the host)
    double v[PER];
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int i = ln() + r * W;
        v[r] = 0.0;
        if (i < L->cv_cells) v[r] = c.T[node[sig[i]]];
    }
    esync();
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int i = ln() + r * W;
        if (i < L->cv_cells) c.T[node[i]] = v[r];
    }
    esync();
}

// ------------------------------------------------------------------ step
// A step's calendar values (row kk before the step, kk - 1 for the comfort
// transition, row j = kk + 1 after it) and aux-time row j. row_issue only
// issues the loads; row_store puts them in a calendar section of the state
// image. The host guarantees j < n1 for every step of an episode.
struct RowVals {
    double v[RW_COUNT];
    double aux;
};

template <int W>
__device__ __forceinline__ RowVals row_issue(const Ctx& c, int kk, int j) {
    const SBK_C DevScen* S = c.S;
    const int naux = c.L->n_aux - 1;
    const int km1 = kk > 0 ? kk - 1 : 0;
    RowVals r;
    r.v[RW_AMB_K] = S->amb[kk];
    r.v[RW_SOLAR_K] = S->solar_i[kk];
    r.v[RW_COMF_K] = S->comfort[kk];
    r.v[RW_COMF_KM1] = kk > 0 ? S->comfort[km1] : 0.0;
    r.v[RW_HSP_K] = S->heat_sp[kk];
    r.v[RW_CSP_K] = S->cool_sp[kk];
    r.v[RW_AMB_J] = S->amb[j];
    r.v[RW_HSP_J] = S->heat_sp[j];
    r.v[RW_CSP_J] = S->cool_sp[j];
    r.v[RW_OCC_HOUR_J] = (double)S->occ_hour[j];
    r.v[RW_OCC_WORK_J] = (double)S->occ_work[j];
    r.v[RW_REW_HOUR_J] = (double)S->rew_hour[j];
    r.v[RW_REW_MONTH_J] = (double)S->rew_month[j];
    r.v[RW_REW_WORK_J] = (double)S->rew_work[j];
    const int l = ln();
    r.aux = naux > 0 ? S->aux_time[(size_t)j * naux + (l < naux ? l : 0)] : 0.0;
    return r;
}

template <int W>
__device__ __forceinline__ void row_store(Ctx& c, const RowVals& r, double* dst) {
    const int l = ln();
    if (l == 0) {
#pragma unroll
        for (int i = 0; i < RW_COUNT; i++) dst[i] = r.v[i];
    }
    if (l < c.L->n_aux - 1) dst[RW_COUNT + l] = r.aux;
}

// The calendar section of calendar index kk.
__device__ __forceinline__ double* cal_section(const Ctx& c, int kk) { return c.cal + (kk & 1) * c.L->st.cal_n; }

// ------------------------------------------------------------------ reset
// sb_sim_reset (sb_sim.c:177-218) on the LDS image; pump head is not reset.
template <int W>
__device__ __forceinline__ void sim_reset(Ctx& c, int start) {
    const SBK_C DevLayout* L = c.L;
    const SBK_C DevScen* S = c.S;
    for (int a = ln(); a < L->na; a += W) {
        const double* ac = c.t.ahu_c() + a * 9;
        c.run[a] = (int)ac[8];
        c.recirc[a] = ac[0];
        c.sat[a] = ac[6];
        c.fan[a] = ac[7];
        c.flow[a] = 0.0;
        c.coolreq[a] = 0;
    }
    for (int v = ln(); v < L->nv; v += W) {
        const double* vc = c.t.vav_c() + v * 9;
        c.damper[v] = vc[7];
        c.reheat[v] = vc[8];
        c.ratio[v] = 1.0;
        c.heatsp[v] = vc[5];
        c.coolsp[v] = vc[6];
        c.mode[v] = M_OFF;
        c.prev_valid[v] = 0;
        c.dcmd_set[v] = 0;
        c.rcmd_set[v] = 0;
        c.dcmd[v] = 0.0;
        c.rcmd[v] = 0.0;
    }
    for (int t = ln(); t < L->n; t += W) {
        c.T[t] = S->temp_init[t];
        c.M[t] = S->mass_init[t];
    }
    if (ln() == 0) {
        c.ip[PI_HWS_REQ] = 0;
        c.ip[PI_HWS_RUN] = 1;
        c.ip[PI_PUMP_RUN] = 1;
        c.plant[PF_BOILER_SP] = S->boiler_c[0];
        c.plant[PF_BOILER_RET] = S->boiler_c[1];
        c.plant[PF_BOILER_CUR] = S->boiler_c[0];
        c.plant[PF_BOILER_DSTEP] = 0.0;
        c.ip[PI_STEP_INDEX] = start;
        c.ip[PI_STEP] = 0;
    }
    esync();
    zone_means<W>(c, c.zq);
    esync();
    for (int v = ln(); v < L->nv; v += W) {
        double area;
        c.sensing[v] = vav_temp(c, c.zq, v, &area);
    }
    esync();
}

// puf_reset sequence (pufferlib_cpu_env.h:187-208) at the env's start offset;
// tail: also zero the observation row's padding (puf_reset, not auto-reset).
template <int W>
__device__ __forceinline__ void env_reset(Ctx& c, int start, float* obs_row, bool tail) {
    const SBK_C DevScen* S = c.S;
    const RowVals first = row_issue<W>(c, start, start + 1);   // the new episode's first step
    sim_reset<W>(c, start);
    // two occupancy intervals around the first observation; one loop body so
    // the (large) occupancy code is emitted once here
#pragma nounroll
    for (int k = 0; k < 2; k++) {
        occupancy_advance<W>(c, k == 0 ? S->hour_m1[start] : S->occ_hour[start],
                             k == 0 ? S->work_m1[start] : S->occ_work[start], c.occ_state, c.occV);
        if (k == 0) write_obs<W>(c, obs_row, S->amb[start], S->aux_time + (size_t)start * (c.L->n_aux - 1), tail);
    }
    row_store<W>(c, first, cal_section(c, start));
    esync();
}


// Action decode and apply (sb_sim.c:557-576, :220-244): continuous actions
// clamp to [-1, 1] and map through float32 (min, max) spans, discrete ones map
// 1 -> max and anything else -> min in float64; the value then goes to its
// host-resolved target. Both decodes are computed and one selected, so lanes
// do not diverge; actions are taken four per lane at a time.
template <int W>
__device__ __forceinline__ void decode_apply(Ctx& c) {
#pragma clang fp contract(off)
    const int n = c.L->n_act;
    const Tab& t = c.t;
    constexpr int U = 4;
    for (int i0 = 0; i0 < n; i0 += U * W) {
        int src[U];
        uint32_t dst[U], aux[U];
        uint8_t disc[U], fl[U];
        double mn[U], mx[U], mnr[U], mxr[U], hi[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * W + ln();
            const int ic = i < n ? i : n - 1;
            src[u] = t.act_src()[ic];
            dst[u] = t.act_dst()[ic];
            aux[u] = t.act_aux()[ic];
            disc[u] = t.act_disc()[ic];
            fl[u] = t.act_flags()[ic];
            mn[u] = t.act_mn()[ic];
            mx[u] = t.act_mx()[ic];
            mnr[u] = t.act_mnr()[ic];
            mxr[u] = t.act_mxr()[ic];
            hi[u] = t.act_hi()[ic];
        }
        float a[U];
#pragma unroll
        for (int u = 0; u < U; u++) a[u] = c.act[src[u]];
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (i0 + u * W >= n) break;   // wave-uniform: slots past the action count
            const int i = i0 + u * W + ln();
            // continuous: clamp, then the float32 span map
            const float m = a[u] > 1.0f ? 1.0f : (a[u] < -1.0f ? -1.0f : a[u]);
            const float span_in = (float)(mxr[u] - mnr[u]);
            const float span_out = (float)(mx[u] - mn[u]);
            const float r = (m - (float)mnr[u]) / span_in * span_out + (float)mn[u];
            double nat = (double)r;
            // discrete: 1 -> +1, else -1, mapped in float64 (only where a lane holds one;
            // discrete actions follow the continuous ones)
            if (__any(disc[u] != 0)) {
                const double m64 = ((double)a[u] == 1.0) ? 1.0 : -1.0;
                const double nat_d = (m64 - mnr[u]) / (mxr[u] - mnr[u]) * (mx[u] - mn[u]) + mn[u];
                nat = disc[u] ? nat_d : nat;
            }
            double v = nat;
            if (fl[u] & ACT_CLAMP) v = nat < 0.0 ? 0.0 : (nat > hi[u] ? hi[u] : nat);
            if (fl[u] & ACT_PUMP_HEAD) v = nat / (GRAV * RHO_W / PA_PER_BAR);
            if (i < n) {
                unsigned char* p = c.envb + (dst[u] & ACT_OFF);
                const int on = (nat == 1.0) ? 1 : 0;
                if (dst[u] & ACT_I32) *reinterpret_cast<int*>(p) = on;
                else *reinterpret_cast<double*>(p) = v;
                unsigned char* q = c.envb + (aux[u] & ACT_OFF);
                if (aux[u] & ACT_AUX_U8) *q = 1;
                if (aux[u] & ACT_AUX_I32) *reinterpret_cast<int*>(q) = on;
            }
        }
    }
    esync();
}

// VAV pass of the pre-step (sb_sim.c:368-384, :316-355, :382-387): sensed
// temperature, thermostat mode, damper and reheat settings, unrestricted flow
// (c.unres by VAV for the column pass, c.lsum at the VAV's position in its
// AHU's list for the AHUs' demand sums), and each VAV's AHU in the register
// slots r = pass * U + u (VAV lane + 64 r) for the flow ratios.
// U VAVs per lane per pass, all loads of a pass before any store.
template <int U>
__device__ __forceinline__ void vav_pass(Ctx& c, int comfort, double& ffs_part, int (&vahu)[SBK_VPL]) {
    const int nv = c.L->nv, lane = ln();
    const double* rw = c.row;
    const double hsp = rw[RW_HSP_K], csp = rw[RW_CSP_K];
    const bool comf_km1 = rw[RW_COMF_KM1] != 0.0;
#pragma unroll
    for (int pass = 0; pass < upasses<U>(); pass++) {
        const int base = pass * 64 * U;
        if (base >= nv) break;
        int v[U], a[U], lp[U], mode[U], pv[U], dset[U], rset[U], run[U];
        bool ok[U];
        double tv[U], area[U], vc0[U], vc1[U], vc2[U], vc4[U], dcmd[U], rcmd[U], dmp[U], rht[U];
        double fan[U], amin[U], varea[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int vv0 = base + 64 * u + lane;
            ok[u] = vv0 < nv;
            v[u] = ok[u] ? vv0 : nv - 1;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            tv[u] = c.sensing[v[u]];
            area[u] = c.fdem[v[u]];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const double* vc = c.t.vav_c() + v[u] * 9;
            vc0[u] = vc[0];
            vc1[u] = vc[1];
            vc2[u] = vc[2];
            vc4[u] = vc[4];
            mode[u] = c.mode[v[u]];
            pv[u] = c.prev_valid[v[u]];
            dset[u] = c.dcmd_set[v[u]];
            rset[u] = c.rcmd_set[v[u]];
            dcmd[u] = c.dcmd[v[u]];
            rcmd[u] = c.rcmd[v[u]];
            dmp[u] = c.damper[v[u]];
            rht[u] = c.reheat[v[u]];
            a[u] = c.t.vav_ahu()[v[u]];
            lp[u] = c.t.vav_lpos()[v[u]];
            varea[u] = c.t.vav_area()[v[u]];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            run[u] = c.run[a[u]];
            fan[u] = c.fan[a[u]];
            amin[u] = c.t.ahu_c()[a[u] * 9 + 2];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const double sensing = tv[u];
            int md = mode[u];
            double damper = dmp[u], reheat = rht[u];
            const bool live = area[u] > 0.0;
            if (live) {
                if (comfort) md = default_mode(md, sensing, hsp, csp);
                else if (pv[u] && comf_km1) md = M_PASSIVE;
                else if (md == M_PASSIVE && sensing > hsp && sensing < csp) md = M_PASSIVE;
                else md = default_mode(md, sensing, hsp, csp);
                double d, h;
                if (md == M_HEAT) { d = 1.0; h = 1.0; }
                else if (md == M_COOL) { d = 1.0; h = 0.0; }
                else { d = vc2[u]; h = 0.0; }
                if (dset[u]) d = dcmd[u];
                if (rset[u]) h = rcmd[u];
                damper = d > vc2[u] ? d : vc2[u];
                reheat = h;
            }
            // unrestricted flow (sb_sim.c:253-265) from the settings just made
            const double st = run[u] != 1 ? 0.0 : (fan[u] > amin[u] ? fan[u] : amin[u]);
            double un = damper * vc0[u] * sqrt(st / vc4[u]);
            un = un > 0.00001 ? un : 0.00001;
            if (ok[u]) {
                if (live) {
                    c.heatsp[v[u]] = hsp;
                    c.coolsp[v[u]] = csp;
                    c.mode[v[u]] = (uint8_t)md;
                    c.prev_valid[v[u]] = 1;
                    c.damper[v[u]] = damper;
                    c.reheat[v[u]] = reheat;
                }
                c.unres[v[u]] = un;
                c.lsum[lp[u]] = un;
                ffs_part += reheat * vc1[u];
                vahu[pass * U + u] = a[u];
            }
        }
    }
}

// Coupled columns (sb_sim.c:410-436, :289-314): reheat energy, air-side
// conductance and supply temperature per column, plus the wavefront's reheat
// total and supply extremes and the register slots for the per-AHU flow sums.
// U columns per lane per pass (lane + 64 u), all loads of a pass issued before
// any store so the U chains overlap; out-of-range slots compute a clamped
// column and drop their results.
template <int U>
__device__ __forceinline__ void coupled_columns(Ctx& c, double ffs, double tf, double iwt, double& total_rw,
                                                double& cmin, double& cmax) {
    const int k = c.L->k;
    const int lane = ln();
#pragma unroll
    for (int pass = 0; pass < upasses<U>(); pass++) {
        const int base = pass * 64 * U;
        if (base >= k) break;
        int col[U], v[U], a[U];
        bool ok[U];
        double area[U], vc0[U], vc1[U], vc3[U], rh[U], dmp[U], un[U], rt[U], sat[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int cc = base + 64 * u + lane;
            ok[u] = cc < k;
            col[u] = ok[u] ? cc : k - 1;
            v[u] = c.t.coupled()[col[u]];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const double* vc = c.t.vav_c() + v[u] * 9;
            area[u] = c.t.vav_area()[v[u]];
            a[u] = c.t.vav_ahu()[v[u]];
            vc0[u] = vc[0];
            vc1[u] = vc[1];
            vc3[u] = vc[3];
            rh[u] = c.reheat[v[u]];
            dmp[u] = c.damper[v[u]];
            un[u] = c.unres[v[u]];
            rt[u] = c.ratio[v[u]];
        }
#pragma unroll
        for (int u = 0; u < U; u++) sat[u] = c.satv[a[u]];
#pragma unroll
        for (int u = 0; u < U; u++) {
            double g = 0.0, ta = 0.0, rw = 0.0, fd = 0.0;
            if (area[u] > 0.0) {
                ta = sat[u];
                fd = un[u] * rt[u];
                // reheat_eff / reheat_energy (sb_sim.c:289-314)
                double eff;
                double air_cap = CP_AIR * RHO_AIR * fd;
                if (air_cap <= 0.0) {
                    eff = 0.0;
                } else {
                    double wflow = 0.0;
                    if (ffs != 0.0) wflow = tf * ((rh[u] * vc1[u]) / ffs);
                    double water_cap = CP_W * RHO_W * wflow;
                    eff = water_cap / air_cap;
                    if (eff > 1.0) eff = 1.0;
                    double gap = iwt - ta;
                    if (gap > 0.0) {
                        double headroom = vc3[u] - ta;
                        if (headroom <= 0.0) eff = 0.0;
                        else {
                            double hr = headroom / gap;
                            if (hr < eff) eff = hr;
                        }
                    }
                }
                rw = eff * CP_AIR * RHO_AIR * fd * (iwt - ta);
                if (dmp[u] > 0.0 && vc0[u] > 0.0) g = fd * RHO_AIR * CP_AIR;
            }
            if (ok[u]) {
                c.g[col[u]] = g;
                c.tair[col[u]] = ta;
                c.rwen[col[u]] = rw;
                c.fdem[c.t.col_lpos()[col[u]]] = fd;
                total_rw += rw;
                cmin = fmin(cmin, ta);
                cmax = fmax(cmax, ta);
            }
        }
    }
}

// Zone heat (sb_sim.c:420-447): the reheat share of each coupled column of
// the zone, internal and occupant gains, per room cell. U zones per lane per
// pass with their column chains interleaved (each zone's columns in order).
template <int U>
__device__ __forceinline__ void zone_heat(Ctx& c, double wpc) {
    const SBK_C DevScen* S = c.S;
    const int nz = c.L->nz;
    const int lane = ln();
#pragma unroll
    for (int pass = 0; pass < upasses<U>(); pass++) {
        const int base = pass * 64 * U;
        if (base >= nz) break;
        int z[U], c0[U], c1[U], ncell[U], occ[U];
        bool ok[U];
        double za[U], q[U];
        int len = 0;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int zz = base + 64 * u + lane;
            ok[u] = zz < nz;
            z[u] = ok[u] ? zz : nz - 1;
            c0[u] = c.t.zone_col_off()[z[u]];
            c1[u] = c.t.zone_col_off()[z[u] + 1];
            ncell[u] = c.t.zone_cell_off()[z[u] + 1] - c.t.zone_cell_off()[z[u]];
            za[u] = c.t.zone_area()[z[u]];
            occ[u] = c.occV[z[u]];
            q[u] = 0.0;
            len = max(len, c1[u] - c0[u]);
        }
        for (int i = 0; i < len; i++) {
            int col[U], v[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                col[u] = c.t.zone_cols()[c0[u] + i < c1[u] ? c0[u] + i : c0[u]];
                v[u] = c.t.coupled()[col[u]];
            }
            double area[U], dmp[U], vc0[U], rw[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                area[u] = c.t.vav_area()[v[u]];
                dmp[u] = c.damper[v[u]];
                vc0[u] = c.t.vav_c()[v[u] * 9];
                rw[u] = c.rwen[col[u]];
            }
#pragma unroll
            for (int u = 0; u < U; u++)
                if (c0[u] + i < c1[u] && area[u] > 0.0 && dmp[u] > 0.0 && vc0[u] > 0.0)
                    q[u] += rw[u] * za[u] / area[u];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            double qq = q[u];
            if (S->internal_w_m2 > 0.0) qq += wpc * (double)ncell[u];
            if (S->occupant_w > 0.0) qq += (double)occ[u] * S->occupant_w;
            if (ok[u]) c.zq[z[u]] = qq / (double)ncell[u];
        }
    }
}

template <int W>
__device__ __forceinline__ void step_pre(Ctx& c, const KParams& P, int* sy) {
    const SBK_C DevLayout* L = c.L;
    const SBK_C DevScen* S = c.S;
    const double* rw = c.row;
    const double ambient = rw[RW_AMB_K];
    const int comfort = (rw[RW_COMF_K] != 0.0);
    const int na = L->na, nv = L->nv;
    // the zone means and VAV sensed temperatures come from the helper
    // wavefront, which computes them while this one decodes the actions
    env_wait(sy + SY_SENS, 1);
    STAMP(12);
    // AHU return-air means and supply temperatures (sb_sim.c:382-387, :253-265):
    // flow-factor sum over all VAVs, then one lane per AHU sums over its VAVs
    // in VAV order (as csim accumulates them)
    double tmean = 0.0;
    if (S->conv_tmean) {
        double s = 0.0;
        for (int t = ln(); t < L->n; t += W) s += c.T[t];
        tmean = bsum<W>(s, c.red) / (double)L->n;
    }
    // sensing, thermostat and VAV settings (sb_sim.c:368-384, :316-355), then
    // this lane's VAVs (v = lane + 64 r) kept in registers for the AHU sums
    double ffs_part = 0.0;
    int vahu[SBK_VPL];
#pragma unroll
    for (int r = 0; r < SBK_VPL; r++) vahu[r] = -1;
    if (nv > 64) vav_pass<2>(c, comfort, ffs_part, vahu);
    else vav_pass<1>(c, comfort, ffs_part, vahu);
    STAMP(13);
    const double ffs = bsum<W>(ffs_part, c.red);
    STAMP(20);
    // each AHU's flow demand: the unrestricted flows of its VAVs, by lane a
    esync();
    int unused_dm;
    const double dm = ahu_sums_of<false>(c.lsum, c.t.ahu_vav_off(), na, unused_dm);
    env_wait(sy + SY_RET, 1);   // the helper's return-air sums
    STAMP(21);
    if (ln() < na) {
        const int a = ln();
        const double ws = c.wsum[a], at = c.atotal[a];
        double rt = (at > 0.0) ? ws / at : tmean;
        double mixed = c.recirc[a] * rt + (1.0 - c.recirc[a]) * ambient;
        c.satv[a] = (mixed > c.sat[a] && c.run[a] == 1) ? c.sat[a] : mixed;
        c.demand[a] = dm;
    }
    if (ln() == 0) {
        c.misc[MS_FFS] = ffs;
        c.ip[PI_HWS_REQ] = nv;
    }
    esync();
    // flow ratio per VAV from its AHU's demand, AHUs from the register slots
    {
        double rt[SBK_VPL];
#pragma unroll
        for (int r = 0; r < SBK_VPL; r++) {
            rt[r] = 1.0;
            if (64 * r < nv) {
                const int a = vahu[r] >= 0 ? vahu[r] : 0;
                const double dm = c.demand[a], mf = c.t.ahu_c()[a * 9 + 1];
                if (dm > 0.0) {
                    const double q = mf / dm;
                    rt[r] = q < 1.0 ? q : 1.0;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < SBK_VPL; r++) {
            const int v = ln() + 64 * r;
            if (64 * r < nv && v < nv) c.ratio[v] = rt[r];
        }
    }
    esync();
    STAMP(14);
    const double tf = total_flow_rate(c);
    const double iwt = c.plant[PF_BOILER_CUR];
    // coupled columns: reheat energy, air-side conductance, AHU flow (sb_sim.c:410-436),
    // and the coil extremes for the boiler return temperature (sb_sim.c:495-499)
    double total_rw = 0.0, cmin = 1e308, cmax = -1e308;
    if (L->k > 64) coupled_columns<2>(c, ffs, tf, iwt, total_rw, cmin, cmax);
    else coupled_columns<1>(c, ffs, tf, iwt, total_rw, cmin, cmax);
    STAMP(22);
    esync();
    // AHU flow (clamped to the AHU's maximum) and cooling requests: by lane a
    // over its columns' flow demands (c.fdem at each column's position in the
    // AHU's list; 0 where the VAV has no zone area), the requests its columns
    // with a demand > 0
    int cnt;
    const double f = ahu_sums_of<true>(c.fdem, c.t.ahu_col_off(), na, cnt);
    wave_sum_min_max(total_rw, cmin, cmax);
    STAMP(23);
    STAMP(24);
    if (ln() < na) {
        const int a = ln();
        const double mf = c.t.ahu_c()[a * 9 + 1];
        c.flow[a] = f > mf ? mf : f;
        c.coolreq[a] = cnt;
    }
    if (ln() == 0) {
        c.misc[MS_TOTAL_REHEAT] = total_rw;
        c.misc[MS_TF] = tf;
        c.misc[MS_CMIN] = cmin;
        c.misc[MS_CMAX] = cmax;
        c.misc[MS_AMB] = ambient;
        c.misc[MS_COMFORT] = comfort;
    }
    // zone heat: reheat share, internal and occupant gains (sb_sim.c:420-447)
    const double frac = comfort ? 1.0 : S->standby_frac;
    const double wpc = S->internal_w_m2 * S->cv_area * frac;
    STAMP(25);
    if (L->nz > 64) zone_heat<2>(c, wpc);
    else zone_heat<1>(c, wpc);
    esync();
}

// ------------------------------------------------------------------ solve plan
struct PassRegs {
    uint64_t h;
    uint32_t w[SBK_KMAX];
    int meta;   // the pass record's field word (wave-uniform, kept in a scalar register)
};

// Pass record fields (nact | maxcnt << 8 | has_pivot << 16 | lgmax << 17;
// lgmax: log2 of the pass's widest segment).
__device__ __forceinline__ int pass_maxcnt(int meta) { return (meta >> 8) & 0xff; }
__device__ __forceinline__ bool pass_pivot(int meta) { return (meta >> 16) & 1; }
__device__ __forceinline__ int pass_lgmax(int meta) { return (meta >> 17) & 7; }

// Issues the loads of one pass's lane header and terms into registers: the
// header of this lane (every lane has one, idle lanes included) and four
// 16-byte words from the lane's start (word_off + lane * stride; idle lanes
// read lane 0's). Words past the lane's stride belong to the next lane or pass
// and are masked when the pass runs, so nothing here waits for a load. The
// record's field word stays in a register, so the pass reads no LDS before its
// terms.
__device__ __forceinline__ void fetch_pass(const SBK_C DevLayout* L, int4 pi, PassRegs& r) {
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const int hdr_off = pi.x, word_off = pi.y;
    r.meta = __builtin_amdgcn_readfirstlane(pi.z);
    const int nact = r.meta & 0xff, stride = (pass_maxcnt(r.meta) + 3) & ~3;
    const int lane = ln();
    r.h = L->hdr[hdr_off + lane];
    const u4v* wp = reinterpret_cast<const u4v*>(L->words + word_off + (lane < nact ? lane : 0) * stride);
#pragma unroll
    for (int q = 0; q < SBK_KMAX / 4; q++) {
        const u4v v = wp[q];
        r.w[4 * q + 0] = v.x;
        r.w[4 * q + 1] = v.y;
        r.w[4 * q + 2] = v.z;
        r.w[4 * q + 3] = v.w;
    }
}

// Waits for a fetched pass here: the empty asm "uses" every loaded register,
// so the compiler places the memory wait at this point instead of at the first
// use inside the pass (where the loads of the passes after it are in flight).
__device__ __forceinline__ void settle_pass(PassRegs& r) {
    asm volatile("" : "+v"(r.h));
#pragma unroll
    for (int m = 0; m < SBK_KMAX; m++) asm volatile("" : "+v"(r.w[m]));
}

// 1/x from the hardware reciprocal and two Newton steps (about 1 ulp).
__device__ __forceinline__ double recip(double x) {
    double r = __builtin_amdgcn_rcp(x);
    double e = fma(-x, r, 1.0);
    r = fma(r, e, r);
    e = fma(-x, r, 1.0);
    return fma(r, e, r);
}

// One group of 4 terms: the slot reads (issued early) and the products
// subtracted in term order. A term word is a | b << 16 (C3 false: the product
// slot[a] * slot[b]) or a | b << 12 | v << 24 (C3: slot[a] * rs[v] * slot[b],
// rs[0] = 1.0 and rs[k + 1] the reciprocal of pivot k, which unscaled L
// entries take when they are read).
template <bool C3>
struct TermGroup {
    double x[4], y[4], z[C3 ? 4 : 1];
};
template <bool C3>
__device__ __forceinline__ void load_terms(const double* slots, const double* rs, const PassRegs& r, int m0,
                                           TermGroup<C3>& g) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t w = r.w[m0 + j];
        if constexpr (C3) {
            g.x[j] = slots[w & 0xfffu];
            g.y[j] = slots[(w >> 12) & 0xfffu];
            g.z[j] = rs[w >> 24];
        } else {
            g.x[j] = slots[w & 0xffffu];
            g.y[j] = slots[w >> 16];
        }
    }
}
template <bool C3>
__device__ __forceinline__ double sub_terms(double acc, const TermGroup<C3>& g) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if constexpr (C3) acc = fma(-(g.x[j] * g.z[j]), g.y[j], acc);
        else acc = fma(-g.x[j], g.y[j], acc);
    }
    return acc;
}

// One pass: every task computes slot[target] = (slot[target] - sum of its
// terms) * slot[mul] on its segment of lanes. Each lane subtracts its own terms
// (the leader from slot[target], the others from 0), a butterfly over the
// segment (lane ^ 1, ^ 2, then the other quad and the other half-row, whose
// lanes hold equal sums by then) gives every lane of the segment the same
// total, and the leader stores it. In a pass holding pivots, lanes also store
// the reciprocal of their result to slot[inv_target] (the sink for non-pivots,
// non-leaders and idle lanes). Terms run in groups of 4 up to the pass's
// longest lane (its stride is that rounded up to 4, so a group never reaches
// another lane's words); terms past a lane's count are (0, 0) and read slot
// 0 = 0.
template <bool C3>
__device__ __forceinline__ void run_pass(double* slots, const double* rs, const PassRegs& r) {
    const int meta = r.meta;
    const int tgt = (int)(r.h & 0xffffu);
    const int mul = (int)((r.h >> 16) & 0xffffu);
    const int invt = (int)((r.h >> 32) & 0xffffu);
    const int flags = (int)(r.h >> 48);
    const int lg = flags & 7;
    const bool lead = (flags >> 3) & 1;
    double acc = slots[tgt];
    const double scale = slots[mul];
    // groups of 4 terms, the reads of the next group issued before the
    // products of the current one (the group count is wave-uniform)
    static_assert(SBK_KMAX == 16, "term groups below are written for 16 terms a lane");
    const int ng = (pass_maxcnt(meta) + 3) >> 2;
    if (ng > 0) {
        TermGroup<C3> ga, gb;
        load_terms<C3>(slots, rs, r, 0, ga);
        if (ng > 1) load_terms<C3>(slots, rs, r, 4, gb);
        acc = sub_terms<C3>(acc, ga);
        if (ng > 1) {
            if (ng > 2) load_terms<C3>(slots, rs, r, 8, ga);
            acc = sub_terms<C3>(acc, gb);
            if (ng > 2) {
                if (ng > 3) load_terms<C3>(slots, rs, r, 12, gb);
                acc = sub_terms<C3>(acc, ga);
                if (ng > 3) acc = sub_terms<C3>(acc, gb);
            }
        }
    }
    // only the butterfly steps the pass's widest segment needs (wave-uniform);
    // every lane of a step's row pattern is a source, so the moves need no
    // fill value
    const int lgmax = pass_lgmax(meta);
    if (lgmax >= 1) {
        double t = dpp_d<DPP_QUAD_1032>(acc, acc);
        acc = lg >= 1 ? acc + t : acc;
        if (lgmax >= 2) {
            t = dpp_d<DPP_QUAD_2301>(acc, acc);
            acc = lg >= 2 ? acc + t : acc;
            if (lgmax >= 3) {
                t = dpp_d<DPP_ROW_HALF_MIRROR>(acc, acc);
                acc = lg >= 3 ? acc + t : acc;
                if (lgmax >= 4) {
                    t = dpp_d<DPP_ROW_MIRROR>(acc, acc);
                    acc = lg >= 4 ? acc + t : acc;
                }
            }
        }
    }
    acc *= scale;
    if (lead) slots[tgt] = acc;
    if (pass_pivot(meta)) slots[invt] = recip(acc);
}

// All passes, in groups of SBK_PLAN_DEPTH (the pass count is a multiple of
// it): a group's loads go out together and its passes wait for their own in
// turn, and the next group's first pass is loaded before the group's last one
// runs. Only that one pass's loads are in flight across the loop's back edge,
// so the compiler's memory waits stay exact (a wait for pass k of a group
// leaves the later passes' loads in flight).
template <int W, bool C3>
__device__ __forceinline__ void run_plan(const SBK_C DevLayout* L, double* slots, const int4* rec,
                                         unsigned long long* pts) {
    static_assert(W == 64, "the solve plan runs on one wavefront");
    constexpr int D = SBK_PLAN_DEPTH;
    const int np = L->n_pass;
    if (np == 0) return;
    const double* rs = slots + L->lu_sbase;
    PassRegs R[D];
    fetch_pass(L, rec[0], R[0]);
    for (int p = 0; p < np; p += D) {
        if (pts) pts[p] = clock64();
#pragma unroll
        for (int k = 1; k < D; k++) fetch_pass(L, rec[p + k], R[k]);
        // the group's loads are issued before the first pass waits for its
        // own (the scheduler may not move them below this point)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < D; k++) {
            if (k == D - 1) {
                fetch_pass(L, rec[min(p + D, np - 1)], R[0]);
                __builtin_amdgcn_sched_barrier(0);
            }
            settle_pass(R[k]);
            run_pass<C3>(slots, rs, R[k]);
            wave_lds_sync();
        }
    }
    if (pts) pts[np] = clock64();
}

// The LU slots' starting values (the permuted matrix, the zero and one slots)
// copied HBM -> LDS in 16-byte vectors, every load of a round (8 KB per
// wavefront) issued before the round's first store, so the copy costs about
// one memory latency per round instead of one per 512 bytes.
__device__ __forceinline__ void copy_slot_init(double* dst, const SBK_C double* src, int count) {
    constexpr int U = 8, W = 64;
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const int n16 = count >> 1, lane = ln();
    const SBK_C u4v* s = reinterpret_cast<const SBK_C u4v*>(src);
    u4v* d = reinterpret_cast<u4v*>(dst);
    for (int base = 0; base < n16; base += U * W) {
        u4v r[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = min(base + u * W + lane, n16 - 1);
            r[u] = s[i];
        }
#pragma unroll
        for (int u = 0; u < U; u++) asm volatile("" : "+v"(r[u]));
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * W + lane;
            if (i < n16) d[i] = r[u];
        }
    }
    if ((count & 1) && lane == 0) dst[count - 1] = src[count - 1];
}

// ------------------------------------------------------------------ relaxation
// (A + diag(g)) y = b by Jacobi sweeps, for layouts whose host-computed bound
// rho = max_i sum_j |a_ij| / a_ii is at most 1/2 (g >= 0 only strengthens the
// diagonal, so rho bounds every step's iteration matrix in the infinity norm).
// Lane l owns rows l, l + 64, l + 128, l + 192: their right-hand sides,
// reciprocal diagonals and off-diagonal entries stay in registers, the iterate
// lives in LDS (in the state image's T array, which starts as the previous
// step's solution). A sweep reads every neighbour value before any lane writes
// (one wavefront; its LDS operations complete in issue order), so it is a true
// Jacobi sweep. It stops once rho / (1 - rho) * max|x_m - x_{m-1}|, a bound on
// the distance to the exact solution, is at most SBK_RX_TOL * max|T|.
// Sweeps with K off-diagonal terms per row (the tables are padded with
// (0.0, column 0) entries, so every load is unconditional and a sweep issues
// all its LDS reads back to back). Returns the number of sweeps.
template <int K>
__device__ __forceinline__ int relax_sweeps(const SBK_C DevLayout* L, double* x, int n, const double* bv,
                                            const double* iv, double* xv, double atol,
                                            unsigned long long* pts) {
    const int lane = ln();
    double av[SBK_RX_RPL][K];
    int ci[SBK_RX_RPL][K];
#pragma unroll
    for (int j = 0; j < SBK_RX_RPL; j++) {
        const int t = lane + 64 * j;   // < SBK_RX_ROWS: tables are padded
#pragma unroll
        for (int m = 0; m < K; m++) {
            av[j][m] = L->rx_val[m * SBK_RX_ROWS + t];
            ci[j][m] = L->rx_col[m * SBK_RX_ROWS + t];
        }
    }
    double stop = L->rx_stop;
    asm volatile("" : "+v"(stop));   // keep it in a VGPR: no scalar reload (and lgkm wait) per sweep
    if (pts) pts[1] = clock64();
    int it = 0;
    bool done = false;
    while (!done) {
        double xn[SBK_RX_RPL];
#pragma unroll
        for (int j = 0; j < SBK_RX_RPL; j++) {
            double acc = bv[j];
#pragma unroll
            for (int m = 0; m < K; m++) acc -= av[j][m] * x[ci[j][m]];
            xn[j] = acc * iv[j];
        }
        double dmax = 0.0;
#pragma unroll
        for (int j = 0; j < SBK_RX_RPL; j++) {
            const int t = lane + 64 * j;
            if (t < n) {
                dmax = fmax(dmax, fabs(xn[j] - xv[j]));
                xv[j] = xn[j];
                x[t] = xn[j];
            }
        }
        wave_lds_sync();
        ++it;
        done = __all(stop * dmax <= atol) || it >= SBK_RX_MAXIT;
        if (pts) pts[1 + it] = clock64();
    }
    return it;
}

template <int W>
__device__ __forceinline__ void relax_solve(Ctx& c, double ambient, double irr, unsigned long long* pts) {
    static_assert(W == 64, "the relaxation sweep runs on one wavefront");
    const SBK_C DevLayout* L = c.L;
    const SBK_C DevScen* S = c.S;
    const int n = L->n;
    const int lane = ln();
    if (pts) pts[0] = clock64();
    double bv[SBK_RX_RPL], iv[SBK_RX_RPL], xv[SBK_RX_RPL];
    double xabs = 0.0;
    // the forcing of this lane's rows: every LDS read issued before the first
    // use, then selects (rows past n read node 0 and rows without an air
    // column read column 0; both are dropped by the selects)
    const uint8_t* isroom = c.t.is_room();
    const double *solar = c.t.solar_c(), *cap = c.t.cap(), *mcoup = c.t.mcoup(), *rxd = c.t.rx_diag();
    const int* rxa = c.t.rx_air();
    int fcol[SBK_RX_RPL];
    uint8_t fr[SBK_RX_RPL];
    double fs[SBK_RX_RPL], fo[SBK_RX_RPL], fc[SBK_RX_RPL], ft[SBK_RX_RPL], fd[SBK_RX_RPL], fm[SBK_RX_RPL],
        fM[SBK_RX_RPL], fdi[SBK_RX_RPL];
#pragma unroll
    for (int j = 0; j < SBK_RX_RPL; j++) {
        const int t = lane + 64 * j < n ? lane + 64 * j : 0;
        fr[j] = isroom[t];
        fs[j] = c.slots[t];
        fo[j] = solar[t];
        fc[j] = cap[t];
        ft[j] = c.T[t];
        fd[j] = c.dirx[t];
        fm[j] = mcoup[t];
        fM[j] = c.M[t];
        fdi[j] = rxd[t];
        fcol[j] = rxa[t];
    }
    double fg[SBK_RX_RPL], fa[SBK_RX_RPL];
#pragma unroll
    for (int j = 0; j < SBK_RX_RPL; j++) {
        const int col = fcol[j] >= 0 ? fcol[j] : 0;
        fg[j] = c.g[col];
        fa[j] = c.tair[col];
    }
#pragma unroll
    for (int j = 0; j < SBK_RX_RPL; j++) {
        const bool ok = lane + 64 * j < n;
        const double qr = fs[j] + fo[j] * irr, qo = fo[j] * irr;
        const double qin = fr[j] ? qr : qo;
        double b = fc[j] * ft[j] + qin + ambient * fd[j] + fm[j] * fM[j];
        double d = fdi[j];
        const bool ha = fcol[j] >= 0;
        const double bg = b + fg[j] * fa[j], dg = d + fg[j];
        b = ha ? bg : b;
        d = ha ? dg : d;
        bv[j] = ok ? b : 0.0;
        iv[j] = ok ? recip(d) : 0.0;
        xv[j] = ok ? ft[j] : 0.0;
        xabs = fmax(xabs, fabs(xv[j]));
    }
    const double atol = SBK_RX_TOL * wave_max(xabs);
    const int nt = L->rx_terms;
    const int it = nt <= 4   ? relax_sweeps<4>(L, c.T, n, bv, iv, xv, atol, pts)
                   : nt <= 6 ? relax_sweeps<6>(L, c.T, n, bv, iv, xv, atol, pts)
                             : relax_sweeps<SBK_RX_TERMS>(L, c.T, n, bv, iv, xv, atol, pts);
    if (lane == 0) {
        c.plant[PF_SWEEPS] = (double)it;
        if (it >= SBK_RX_MAXIT) c.plant[PF_CAPPED] += 1.0;
    }
#pragma unroll
    for (int j = 0; j < SBK_RX_RPL; j++) {
        const int t = lane + 64 * j;
        if (t < n) c.M[t] = c.M[t] * c.t.mret()[t] + c.t.mgain()[t] * xv[j];
    }
    esync();
}

// ------------------------------------------------------------------ block relaxation
// Block-Jacobi form: lane l owns blocks l and l + 64 (block slot q < Q) of at
// most three nodes. Once per step each block's matrix A_BB + G_B is inverted
// in registers (Gauss-Jordan without pivoting: it is an M-matrix, so pivots
// stay positive) and folded into the block's list of off-block entries:
//   x_B = c0 - sum_t cf_t x[col_t],  c0 = (A_BB + G_B)^-1 b_B,
//   cf_t = (A_BB + G_B)^-1 e_{row_t} a_t,
// so a sweep is one LDS gather per off-block entry and a few FMAs per row.
// Padding rows have c0 = cf = 0 and store to a per-lane sink. Same stopping
// bound as the point form, with the host's block rho.
constexpr int BXR = SBK_BX_ROWS, BXT = SBK_BX_TERMS;

template <int Q>
__device__ __forceinline__ int block_sweeps(double* x, const int (&col)[Q][BXT], const double (&cf)[Q][BXR][BXT],
                                            const double (&c0)[Q][BXR], const int (&dst)[Q][BXR],
                                            double (&xv)[Q][BXR], double stop, double atol,
                                            unsigned long long* pts) {
    asm volatile("" : "+v"(stop));   // keep it in a VGPR: no scalar reload (and lgkm wait) per sweep
    if (pts) pts[1] = clock64();
    int it = 0;
    bool done = false;
    while (!done) {
        double xg[Q][BXT];
#pragma unroll
        for (int q = 0; q < Q; q++) {
#pragma unroll
            for (int t = 0; t < BXT; t++) xg[q][t] = x[col[q][t]];
        }
        double dmax = 0.0;
#pragma unroll
        for (int q = 0; q < Q; q++) {
#pragma unroll
            for (int p = 0; p < BXR; p++) {
                double acc = c0[q][p];
#pragma unroll
                for (int t = 0; t < BXT; t++) acc -= cf[q][p][t] * xg[q][t];
                dmax = fmax(dmax, fabs(acc - xv[q][p]));
                xv[q][p] = acc;
            }
        }
#pragma unroll
        for (int q = 0; q < Q; q++) {
#pragma unroll
            for (int p = 0; p < BXR; p++) x[dst[q][p]] = xv[q][p];
        }
        wave_lds_sync();
        ++it;
        done = __all(stop * dmax <= atol) || it >= SBK_RX_MAXIT;
        if (pts) pts[1 + it] = clock64();
    }
    return it;
}

template <int Q>
__device__ __forceinline__ void relax_block_solve(Ctx& c, double ambient, double irr, unsigned long long* pts) {
    const SBK_C DevLayout* L = c.L;
    const int lane = ln();
    if (pts) pts[0] = clock64();
    // per-lane sink for padding rows, as an index relative to the iterate
    const int sink = (int)((c.red + lane) - c.T);
    // block tables from the staged layout image: lane l takes block q * 64 + l
    // (clamped into the table, and then turned into padding, past the last one)
    static_assert(BXR == 3 && BXT == 8, "the chunk layout holds three rows and eight entries");
    const int nb = L->bx_nb;
    const double2* bxd = reinterpret_cast<const double2*>(c.imgb + L->img.bx_d);
    const int4* bxi = reinterpret_cast<const int4*>(c.imgb + L->img.bx_i);
    int row[Q][BXR], col[Q][BXT];
    int dst[Q][BXR];
    double xv[Q][BXR], c0[Q][BXR], cf[Q][BXR][BXT];
    double xabs = 0.0;
    // the forcing b = cap T + q + amb dirx + mc M of every node into the slot
    // region (which holds each room cell's zone heat), node-major: lane l
    // takes nodes l + 64 j, three per round with every read of a round
    // issued before the first use (n <= 192 Q: every node sits in one of at
    // most 64 Q blocks of at most three)
    {
        const int n = L->n;
        const uint8_t* isroom = c.t.is_room();
        const double *solar = c.t.solar_c(), *cap = c.t.cap(), *mcoup = c.t.mcoup();
        constexpr int NR = 3;
#pragma unroll
        for (int j0 = 0; j0 < BXR * Q; j0 += NR) {
            if (64 * j0 >= n) break;
            uint8_t fr[NR];
            double fs[NR], fo[NR], fc[NR], ft[NR], fd[NR], fm[NR], fM[NR];
#pragma unroll
            for (int j = 0; j < NR; j++) {
                const int t0 = lane + 64 * (j0 + j);
                const int t = t0 < n ? t0 : 0;
                fr[j] = isroom[t];
                fs[j] = c.slots[t];
                fo[j] = solar[t];
                fc[j] = cap[t];
                ft[j] = c.T[t];
                fd[j] = c.dirx[t];
                fm[j] = mcoup[t];
                fM[j] = c.M[t];
            }
#pragma unroll
            for (int j = 0; j < NR; j++) {
                const int t0 = lane + 64 * (j0 + j);
                const double qr = fs[j] + fo[j] * irr, qo = fo[j] * irr;
                const double qin = fr[j] ? qr : qo;
                const double bb = fc[j] * ft[j] + qin + ambient * fd[j] + fm[j] * fM[j];
                if (t0 < n) c.slots[t0] = bb;
            }
        }
        esync();
        // the air side: b += g T_air at each column's node (every node has
        // at most one column)
        const int k = L->k;
        const int* an = c.t.air_node();
#pragma unroll
        for (int c0i = 0; c0i < 2; c0i++) {
            if (64 * c0i >= k) break;
            const int cc0 = lane + 64 * c0i;
            const int cc = cc0 < k ? cc0 : 0;
            const int node = an[cc];
            const double gv = c.g[cc], tv = c.tair[cc];
            const double bb = c.slots[node];
            const double bg = bb + gv * tv;
            if (cc0 < k) c.slots[node] = bg;
        }
        esync();
    }
    // one slot at a time (its tables, then its rows' forcing, conductance and
    // temperature, then its matrix)
#pragma unroll
    for (int q = 0; q < Q; q++) {
        int air[BXR], trow[BXT];
        double dia[BXR], inm[BXR][BXR], val[BXT];
        const int blk = q * 64 + lane;
        const bool ok = blk < nb;
        const int bc = ok ? blk : nb - 1;
        double rd[18];
        int ri[12];
#pragma unroll
        for (int j = 0; j < 9; j++) {
            const double2 v = bxd[j * nb + bc];
            rd[2 * j] = v.x;
            rd[2 * j + 1] = v.y;
        }
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const int4 v = bxi[j * nb + bc];
            ri[4 * j] = v.x;
            ri[4 * j + 1] = v.y;
            ri[4 * j + 2] = v.z;
            ri[4 * j + 3] = v.w;
        }
#pragma unroll
        for (int p = 0; p < BXR; p++) {
            row[q][p] = ok ? (ri[p] << 16) >> 16 : -1;
            air[p] = ok ? ri[p] >> 16 : -1;
            dia[p] = ok ? rd[p] : 1.0;
            inm[p][p] = 0.0;
        }
        inm[0][1] = ok ? rd[3] : 0.0;
        inm[0][2] = ok ? rd[4] : 0.0;
        inm[1][0] = ok ? rd[5] : 0.0;
        inm[1][2] = ok ? rd[6] : 0.0;
        inm[2][0] = ok ? rd[7] : 0.0;
        inm[2][1] = ok ? rd[8] : 0.0;
#pragma unroll
        for (int t = 0; t < BXT; t++) {
            val[t] = ok ? rd[9 + t] : 0.0;
            col[q][t] = ok ? ri[4 + t] & 0xffff : 0;
            trow[t] = ok ? ri[4 + t] >> 16 : 0;
        }
        // padding rows read node 0 and rows without an air column column 0;
        // the selects drop both
        double fb[BXR], fg[BXR], ft[BXR];
#pragma unroll
        for (int p = 0; p < BXR; p++) {
            const int tc = row[q][p] >= 0 ? row[q][p] : 0;
            const int ac = air[p] >= 0 ? air[p] : 0;
            fb[p] = c.slots[tc];
            fg[p] = c.g[ac];
            ft[p] = c.T[tc];
        }
        double m[BXR][BXR], bi[BXR][BXR], b[BXR];
#pragma unroll
        for (int p = 0; p < BXR; p++) {
            const int t = row[q][p];
            const double dg = dia[p] + fg[p];
            const double d = air[p] >= 0 ? dg : dia[p];
#pragma unroll
            for (int p2 = 0; p2 < BXR; p2++) {
                m[p][p2] = p2 == p ? d : inm[p][p2];
                bi[p][p2] = p2 == p ? 1.0 : 0.0;
            }
            dst[q][p] = t >= 0 ? t : sink;
            b[p] = t >= 0 ? fb[p] : 0.0;
            xv[q][p] = t >= 0 ? ft[p] : 0.0;
            xabs = fmax(xabs, fabs(xv[q][p]));
        }
        {
            // the inverse as adjugate / determinant (one reciprocal; the block
            // is an M-matrix, so the determinant is positive and the cofactor
            // differences do not cancel badly)
            double adj[BXR][BXR];
#pragma unroll
            for (int i = 0; i < BXR; i++) {
#pragma unroll
                for (int j = 0; j < BXR; j++) {
                    const int r0 = (j + 1) % 3, r1 = (j + 2) % 3, c0i = (i + 1) % 3, c1i = (i + 2) % 3;
                    adj[i][j] = m[r0][c0i] * m[r1][c1i] - m[r0][c1i] * m[r1][c0i];
                }
            }
            const double det = m[0][0] * adj[0][0] + m[0][1] * adj[1][0] + m[0][2] * adj[2][0];
            const double rd = recip(det);
#pragma unroll
            for (int i = 0; i < BXR; i++) {
#pragma unroll
                for (int j = 0; j < BXR; j++) bi[i][j] = adj[i][j] * rd;
            }
        }
#pragma unroll
        for (int p = 0; p < BXR; p++) {
            double acc = 0.0;
#pragma unroll
            for (int p2 = 0; p2 < BXR; p2++) acc += bi[p][p2] * b[p2];
            c0[q][p] = acc;
        }
        // cf = bi * (entry value placed in its row): three plain selects and
        // nine FMAs per entry (a select chain over the row index compiles to
        // exec-mask branches)
#pragma unroll
        for (int t = 0; t < BXT; t++) {
            const int r = trow[t];
            double vr[BXR];
#pragma unroll
            for (int p2 = 0; p2 < BXR; p2++) vr[p2] = r == p2 ? val[t] : 0.0;
#pragma unroll
            for (int p = 0; p < BXR; p++) {
                double acc = bi[p][0] * vr[0];
#pragma unroll
                for (int p2 = 1; p2 < BXR; p2++) acc = fma(bi[p][p2], vr[p2], acc);
                cf[q][p][t] = acc;
            }
        }
    }
    static_assert(BXR == 3, "the entry-row select above assumes three rows per block");
    const double atol = SBK_RX_TOL * wave_max(xabs);
    const int it = block_sweeps<Q>(c.T, col, cf, c0, dst, xv, L->rx_stop, atol, pts);
    if (lane == 0) {
        c.plant[PF_SWEEPS] = (double)it;
        if (it >= SBK_RX_MAXIT) c.plant[PF_CAPPED] += 1.0;
    }
#pragma unroll
    for (int q = 0; q < Q; q++) {
#pragma unroll
        for (int p = 0; p < BXR; p++) {
            const int t = row[q][p];
            if (t >= 0) c.M[t] = c.M[t] * c.t.mret()[t] + c.t.mgain()[t] * xv[q][p];
        }
    }
    esync();
}

// Field step: b = cap T + q + amb dirx + mc M (+ solar, + g T_air at the air
// nodes), then (A + diag(g)) y = b by the plan (or by relaxation); mass and
// field update.
template <int W, int KV>
__device__ __forceinline__ void field_step(Ctx& c, const KParams& P, int* sy) {
    const SBK_C DevLayout* L = c.L;
    const SBK_C DevScen* S = c.S;
    const double ambient = c.row[RW_AMB_K];
    const double irr = c.row[RW_SOLAR_K];
    const int n = L->n;
    double* slots = c.slots;
    if constexpr (KV != KV_LU) {
        // room cells carry their zone's heat (node-indexed scratch in the slot region)
        for (int z = ln(); z < L->nz; z += W) {
            double qz = c.zq[z];
            for (int t = c.t.zone_cell_off()[z]; t < c.t.zone_cell_off()[z + 1]; t++) slots[c.t.zone_cells()[t]] = qz;
        }
        esync();
        STAMP(5);
        unsigned long long* pts = (P.pass_ts && c.e == P.pass_ts_env && ln() == 0) ? P.pass_ts : nullptr;
        if constexpr (KV == KV_BLOCK) {
            if (L->rx_block == 2) relax_block_solve<2>(c, ambient, irr, pts);
            else relax_block_solve<1>(c, ambient, irr, pts);
        } else {
            relax_solve<W>(c, ambient, irr, pts);
        }
        STAMP(6);
        return;
    } else {
    const int vb = L->vec_base;
    env_wait(sy + SY_SLOTS, 1);   // the helper's copy of the slots' starting values [0, vb)
    // room cells carry their zone's heat; every node then gets its solar gain
    for (int z = ln(); z < L->nz; z += W) {
        double qz = c.zq[z];
        for (int t = c.t.zone_cell_off()[z]; t < c.t.zone_cell_off()[z + 1]; t++) c.slots[vb + c.t.pos()[c.t.zone_cells()[t]]] = qz;
    }
    esync();
    for (int t = ln(); t < n; t += W) {
        const int ps = vb + c.t.pos()[t];
        double qin = c.t.is_room()[t] ? slots[ps] + c.t.solar_c()[t] * irr : c.t.solar_c()[t] * irr;
        slots[ps] = c.t.cap()[t] * c.T[t] + qin + ambient * c.dirx[t] + c.t.mcoup()[t] * c.M[t];
    }
    esync();
    for (int col = ln(); col < L->k; col += W) {
        double g = c.g[col];
        slots[c.t.air_slot()[col]] += g;
        slots[vb + c.t.pos()[c.t.air_node()[col]]] += g * c.tair[col];
    }
    esync();
    STAMP(5);
    // level schedule: LU of the permuted system, forward and backward solves
    unsigned long long* pts = (P.pass_ts && c.e == P.pass_ts_env && ln() == 0) ? P.pass_ts : nullptr;
    if (L->lu_sbase) run_plan<W, true>(L, slots, reinterpret_cast<const int4*>(c.prec), pts);
    else run_plan<W, false>(L, slots, reinterpret_cast<const int4*>(c.prec), pts);
    STAMP(6);
    for (int t = ln(); t < n; t += W) {
        double y = slots[vb + c.t.pos()[t]];
        c.M[t] = c.M[t] * c.t.mret()[t] + c.t.mgain()[t] * y;
        c.T[t] = y;
    }
    esync();
    }
}

// sb_sim_step_post (sb_sim.c:489-521), convection off.
template <int W>
__device__ __forceinline__ void step_post(Ctx& c) {
    if (ln() == 0) {
        const SBK_C DevScen* S = c.S;
        const double total_rw = c.misc[MS_TOTAL_REHEAT];
        double wcap = CP_W * RHO_W * c.misc[MS_TF];
        if (wcap > 0.0 && c.L->k > 0) {
            double supply = c.plant[PF_BOILER_CUR];
            double rt = supply - total_rw / wcap;
            double at = total_rw >= 0.0 ? c.misc[MS_CMIN] : c.misc[MS_CMAX];
            double lo = supply < at ? supply : at;
            double hi = supply > at ? supply : at;
            if (rt < lo) rt = lo;
            if (rt > hi) rt = hi;
            c.plant[PF_BOILER_RET] = rt;
        }
        double begin = c.plant[PF_BOILER_CUR], sp = c.plant[PF_BOILER_SP];
        double dt_min = S->dt_sec / 60.0;
        double cur;
        if (sp > begin) {
            double v = begin + S->boiler_c[2] * dt_min;
            cur = v < sp ? v : sp;
        } else if (sp < begin) {
            double v = begin - S->boiler_c[3] * dt_min;
            cur = v > sp ? v : sp;
        } else {
            cur = sp;
        }
        c.plant[PF_BOILER_CUR] = cur;
        c.plant[PF_BOILER_DSTEP] = cur - begin;
        c.ip[PI_STEP_INDEX] += 1;
    }
    esync();
}

// 3C reward (sb_reward.c:31-155) on the post-step state and new occupancy.
// VAV temperatures of the reward's AHU terms (sb_reward.c:62-98): temperature
// * area into c.unres at the VAV's position in its AHU's list (the pre-step's
// scratch, free by now); the areas' per-AHU sums are a layout table.
template <int U>
__device__ __forceinline__ void reward_vavs(Ctx& c, const double* zm) {
    const int nv = c.L->nv, lane = ln();
#pragma unroll
    for (int pass = 0; pass < upasses<U>(); pass++) {
        const int base = pass * 64 * U;
        if (base >= nv) break;
        int v[U];
        bool ok[U];
        double tv[U], area[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int vv0 = base + 64 * u + lane;
            ok[u] = vv0 < nv;
            v[u] = ok[u] ? vv0 : nv - 1;
        }
        vav_temps<U>(c, zm, v, tv, area);
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (ok[u]) c.unres[c.t.vav_lpos()[v[u]]] = tv[u] * area[u];
        }
    }
}

// The reward is computed in two halves on the env's two wavefronts, each on
// its own zone means of the post-step field: the AHU half (blower and cooling
// power) and the rest (boiler gas, pump, occupant productivity), combined by
// reward_combine in csim's order of operations.
struct RewardPart {
    double gas_rate, pump_e, total_occ, cum;
    double dev_sum, dev_max, oob;   // comfort diagnostics: zone deviations from the band
};
static_assert(sizeof(RewardPart) == 4 * (SY_RET - SY_PART), "the helper's reward half fills SY_PART..SY_RET");

// AHU half (sb_reward.c:62-98): `zm` holds the zone means of the post-step
// field. Returns blower (intake + exhaust) and cooling power.
template <int W>
__device__ __forceinline__ void reward_ahu(Ctx& c, const double* zm, double& blower, double& cooling) {
    const SBK_C DevLayout* L = c.L;
    const SBK_C DevScen* S = c.S;
    const double ambient = c.row[RW_AMB_J];
    double tmean = 0.0;
    if (S->conv_tmean) {
        double s = 0.0;
        for (int t = ln(); t < L->n; t += W) s += c.T[t];
        tmean = bsum<W>(s, c.red) / (double)L->n;
    }
    // VAV temperatures (lanes over VAVs), then one lane per AHU: return-air
    // mean over its VAVs in VAV order and its blower / cooling terms, which
    // every lane then sums in AHU order (sb_reward.c:62-98)
    if (L->nv > 64) reward_vavs<2>(c, zm);
    else reward_vavs<1>(c, zm);
    esync();
    int unused;
    const double ws = ahu_sums_of<false>(c.unres, c.t.ahu_vav_off(), L->na, unused);
    if (ln() < L->na) {
        const int a = ln();
        const double at = c.t.ahu_area()[a];
        double rc = (at > 0.0) ? ws / at : tmean;
        double st = ahu_static(c, a);
        double fe = c.t.ahu_c()[a * 9 + 5];
        double flow = (c.run[a] == 1) ? c.flow[a] : 0.0;
        double mixed = c.recirc[a] * rc + (1.0 - c.recirc[a]) * ambient;
        double sat = (mixed > c.sat[a] && c.run[a] == 1) ? c.sat[a] : mixed;
        c.wsum[a] = flow * st / fe;
        c.atotal[a] = flow * (1.0 - c.recirc[a]) * st / fe;
        c.fdsum[a] = flow * RHO_AIR * CP_AIR * (sat - mixed) / c.t.ahu_c()[a * 9 + 4];
    }
    esync();
    double intake = 0.0, exhaust = 0.0, cool = 0.0;
    for (int a = 0; a < L->na; a++) {
        intake += c.wsum[a];
        exhaust += c.atotal[a];
        cool += c.fdsum[a];
    }
    blower = intake + exhaust;
    cooling = cool;
}

// The rest (sb_reward.c:12-29, :99-130): boiler gas rate (log(r2/c6)/c8 +
// 1/c4/r2 precomputed on the host), pump power and the occupant productivity
// sums over zones (`zm` zone means of the post-step field, `occ_v` the new
// occupant counts).
template <int W>
__device__ __forceinline__ RewardPart reward_rest(Ctx& c, const double* zm, const uint8_t* occ_v) {
    const SBK_C DevLayout* L = c.L;
    const SBK_C DevScen* S = c.S;
    const double dt = S->dt_sec, inv_hour = 1.0 / 3600.0;
    const double* rw = c.row;
    const double ambient = rw[RW_AMB_J];
    const double tf = total_flow_rate(c);
    RewardPart out;
    {
        const double* bc = S->boiler_c;
        double rwt = c.plant[PF_BOILER_RET];
        double bsp = c.plant[PF_BOILER_SP];
        double supply = (bsp > rwt) ? bsp : rwt;
        double flow = CP_W * RHO_W * tf * (supply - rwt);
        double diss = 0.0;
        if (supply >= ambient) diss = bc[5] * 2.0 * PI_D * (supply - ambient) / S->diss_den;
        double tank = 0.0;
        if (dt > 0.0) tank = CP_W * RHO_W * bc[7] * c.plant[PF_BOILER_DSTEP] / dt;
        double tot = flow + diss + tank;
        out.gas_rate = tot > 0.0 ? tot : 0.0;
    }
    out.pump_e = tf * RHO_W * GRAV * c.plant[PF_PUMP_HEAD] / S->pump_eff;
    const double max_pph = S->rw[0], ref = S->rw[2];
    const double hsp = rw[RW_HSP_J], csp = rw[RW_CSP_J];
    double occ_part = 0.0, cum_part = 0.0, dsum = 0.0, dmax = 0.0, noob = 0.0;
    {
        // zones z = lane + 64 r: loads of every slot first, then the sums in
        // slot order
        double occv[SBK_VPL], ztv[SBK_VPL];
#pragma unroll
        for (int r = 0; r < SBK_VPL; r++) {
            const int z = ln() + 64 * r;
            const int zc = z < L->nz ? z : 0;
            occv[r] = 0.0;
            ztv[r] = 0.0;
            if (64 * r < L->nz) {
                occv[r] = (double)occ_v[zc];
                ztv[r] = zm[zc];
            }
        }
#pragma unroll
        for (int r = 0; r < SBK_VPL; r++) {
            const int z = ln() + 64 * r;
            if (64 * r < L->nz && z < L->nz) {
                const double occ = occv[r];
                occ_part += occ;
                const double zt = ztv[r];
                double dev = zt - csp;
                if (hsp - zt > dev) dev = hsp - zt;
                if (dev < 0.0) dev = 0.0;
                dsum += dev;
                dmax = fmax(dmax, dev);
                noob += dev > 0.0 ? 1.0 : 0.0;
                double sh = (dev <= ref) ? dev / ref : 1.0 + ((dev - ref) / ref) * ((dev - ref) / ref);
                cum_part += max_pph * (1.0 - sh) * occ * dt * inv_hour;
            }
        }
    }
    wave_sum4_max(occ_part, cum_part, dsum, noob, dmax);
    out.total_occ = occ_part;
    out.cum = cum_part;
    out.dev_sum = dsum;
    out.dev_max = dmax;
    out.oob = noob;
    return out;
}

// Normalised productivity, cost and carbon, and the weighted reward
// (sb_reward.c:99-155).
// The step's 8 diagnostics of the reference GPU env (sb_gpu_kernels.cuh:1466-1473).
struct StepParts {
    double v[8];
};

__device__ __forceinline__ double reward_combine(const Ctx& c, double blower, double cooling, const RewardPart& p,
                                                 StepParts& sp) {
    const SBK_C DevScen* S = c.S;
    const double dt = S->dt_sec, inv_hour = 1.0 / 3600.0;
    const double* rw = c.row;
    const int hour = (int)rw[RW_REW_HOUR_J], month = (int)rw[RW_REW_MONTH_J], wd = (int)rw[RW_REW_WORK_J];
    const double max_pph = S->rw[0], min_pph = S->rw[1];
    const double total_occ = p.total_occ, cum = p.cum;
    const double max_prod = max_pph * total_occ * dt * inv_hour;
    const double min_prod = min_pph * total_occ * dt * inv_hour;
    double npr = 0.0;
    if (total_occ > 0.0 && (max_prod - min_prod) != 0.0) npr = (cum - min_prod) / (max_prod - min_prod) - 1.0;
    const double elec_rate = blower + fabs(cooling) + p.pump_e;
    const double price = wd ? c.elec_wk[hour] : c.elec_we[hour];
    const double crate = c.elec_co2[hour];
    const double elec_cost = price * fabs(elec_rate) * dt;
    const double elec_cost_max = price * S->rw[3] * dt;
    const double elec_carb = crate * fabs(elec_rate) * dt;
    const double elec_carb_max = crate * S->rw[3] * dt;
    const double gprice = c.gas_price[month - 1];
    const double gg = p.gas_rate > 0.0 ? p.gas_rate : 0.0;
    const double gas_cost = gprice * gg * dt;
    const double gas_cost_max = gprice * S->rw[4] * dt;
    const double gas_carb = S->gas_co2 * gg * dt;
    const double gas_carb_max = S->gas_co2 * S->rw[4] * dt;
    const double den_e = elec_cost_max + gas_cost_max;
    const double nec = (den_e > 0.0) ? (elec_cost + gas_cost) / den_e : 0.0;
    const double den_c = elec_carb_max + gas_carb_max;
    const double ncar = (den_c > 0.0) ? (elec_carb + gas_carb) / den_c : 0.0;
    const double pw = S->rw[5], ew = S->rw[6], cw = S->rw[7];
    const double raw = npr * pw - nec * ew - ncar * cw;
    sp.v[0] = npr;
    sp.v[1] = nec;
    sp.v[2] = ncar;
    sp.v[3] = p.dev_sum * S->inv_nz;
    sp.v[4] = p.dev_max;
    sp.v[5] = p.oob * S->inv_nz;
    sp.v[6] = fabs(elec_rate) * S->kwh_per_w;
    sp.v[7] = gg * S->kwh_per_w;
    return raw / (pw + ew + cw);
}

// Store of bytes [begin, end) (16-byte multiples) of the state image back to
// its HBM record, 16 bytes per lane.
template <int W>
__device__ __forceinline__ void store16(unsigned char* dst, const unsigned char* src, int begin, int end) {
    // streaming stores: the record is read back only by the next step's burst
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    for (int i = (begin >> 4) + ln(); i < (end >> 4); i += W)
        __builtin_nontemporal_store(reinterpret_cast<const u4v*>(src)[i], reinterpret_cast<u4v*>(dst) + i);
}

// Staging burst: every thread issues all loads of a round (up to U vectors of
// each part) before its first store, so the burst costs one memory latency
// per round. Indices are clamped into the part (to vector 0 of a valid buffer
// when the part is empty), so every load is unconditional and in bounds.
template <int U, class Src>
__device__ __forceinline__ void part_load(uint4 (&r)[U], Src src, int n16, int tid, int nthr, int base) {
    const int last = n16 > 0 ? n16 - 1 : 0;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int i = base + u * nthr + tid;
        r[u] = src[i < last ? i : last];
    }
}

// Marks the loaded vectors as used here, so the compiler cannot sink each load
// down to its (conditional) store and wait for it there: every load of the
// round is issued before the first wait.
template <int U>
__device__ __forceinline__ void part_pin(uint4 (&r)[U]) {
#pragma unroll
    for (int u = 0; u < U; u++) asm volatile("" : "+v"(r[u].x), "+v"(r[u].y), "+v"(r[u].z), "+v"(r[u].w));
}

template <int U>
__device__ __forceinline__ void part_store(const uint4 (&r)[U], uint4* dst, int n16, int tid, int nthr, int base) {
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int i = base + u * nthr + tid;
        if (i < n16) dst[i] = r[u];
    }
}

// Copies this wavefront's phase stamps to the host-visible array.
__device__ __forceinline__ void stamps_flush(const KParams& P, const Ctx& c) {
    if (!P.phase_ts) return;
    esync();
    const int i = ln();
    if (i < SBK_NSTAMP && c.helper == stamp_is_helpers(i))
        P.phase_ts[(size_t)c.e * SBK_NSTAMP + i] = c.stamps[i];
}


// A whole episode's sums added to the env's host-visible Log (the reference GPU
// env's finalize_k, complete_port/gpu/smart_buildings.cu:2002-2036): each
// field read and written with system-scope accesses (the trainer may clear the
// Log between steps). ep: EP_* running sums, st: the episode's length.
__device__ __forceinline__ void log_episode(const KParams& P, int e, const float* ep, int st) {
    // Log field i by lane i, so the 13 read-modify-writes over the host link
    // are in flight together
    const int i = ln();
    if (i >= 13) return;
    const float s = (float)st;
    float a;
    switch (i) {
    case 0: case 1: a = ep[EP_RET] / s; break;          // perf, score: the episode's mean reward
    case 2: a = ep[EP_RET]; break;
    case 3: a = s; break;
    case 4: a = ep[EP_PART + 3] / s; break;             // comfort_dev_K
    case 5: a = ep[EP_WORST]; break;
    case 6: a = ep[EP_PART + 5] / s; break;             // out_of_band_frac
    case 7: case 8: case 9: a = ep[EP_PART + i - 7] / s; break;   // productivity, energy cost, carbon
    case 10: case 11: a = ep[EP_PART + i - 4]; break;   // elec_kwh, gas_kwh
    default: a = 1.0f; break;                           // n
    }
    float* f = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(P.host_env) + (size_t)e * P.env_stride
                                        + P.log_offset) + i;
    const float x = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(f, x + a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
static_assert(sizeof(Log) == 52 && offsetof(Log, comfort_dev_K) == 16 && offsetof(Log, n) == 48,
              "log_episode writes the reference GPU env's Log field order");

// The env's second wavefront during a step. The occupancy interval is
// exogenous (it reads only the chain states, the MT stream and the calendar),
// so it runs while the first wavefront decodes and runs the HVAC pre-step.
// The observation reads nothing the field solve writes (the post-step boiler
// update does not read the field either, so the first wavefront runs it before
// the solve), so it is written while the first wavefront solves; the new chain
// states are committed after it has read the old counts. Once the field is
// there, the reward's non-AHU half (gas, pump, productivity and the comfort
// diagnostics) goes to the first wavefront, which computes the AHU half
// meanwhile. Each wait is for a post the first wavefront always makes.
template <int W, int KV>
__device__ __forceinline__ void helper_step(Ctx& c, const KParams& P, int* sy, unsigned char* env, float* obs_row,
                                            int kk, int j) {
    const SBK_C DevLayout* L = c.L;
    const int nocc = L->nz * L->nassign;

    // zone means and VAV sensed temperatures of the field before the step,
    // while the first wavefront decodes the actions
    zone_means<W>(c, c.zq);
    esync();
    {
        if (L->nv > 64) vav_sensing<2>(c);
        else vav_sensing<1>(c);
        env_post(sy + SY_SENS, 1);
        // each AHU's return-air sums over its VAVs in VAV order (sb_sim.c:
        // 382-387) by lane a, for the first wavefront's supply temperatures
        // (c.wsum / c.atotal: reward scratch, free until then)
        esync();
        int unused;
        const double ws = ahu_sums_of<false>(c.rwen, c.t.ahu_vav_off(), L->na, unused);
        if (ln() < L->na) {
            c.wsum[ln()] = ws;
            c.atotal[ln()] = c.t.ahu_area()[ln()];
        }
        env_post(sy + SY_RET, 1);
    }
    if constexpr (KV == KV_LU) {
        // the LU slots' starting values (the permuted matrix, the zero and
        // one slots), copied while the first wavefront runs the pre-step; its
        // field step waits for this post instead of copying them
        copy_slot_init(c.slots, L->slot_init, L->vec_base);
        env_post(sy + SY_SLOTS, 1);
    }
    uint8_t* st_new = env + L->lds.occn;
    uint8_t* v_new = st_new + nocc;
    const bool occ_twisted = occupancy_advance<W>(c, (int)c.row[RW_OCC_HOUR_J], (int)c.row[RW_OCC_WORK_J], st_new,
                                                  v_new);
    if (c.conv) {
        conv_plan<W>(c, occ_twisted);
        env_post(sy + SY_CONV, 1);
    }
    STAMP(15);
    {
        // the next step's calendar values (rows kk + 1 and j + 1) into the
        // other calendar section of the state image, loaded while this
        // wavefront waits for the pre-step state; after the last step of an
        // episode the reset path writes the new episode's own, so clamping to
        // the tables is enough there
        const int n1 = c.S->n1;
        const RowVals next = row_issue<W>(c, min(kk + 1, n1 - 1), min(j + 1, n1 - 1));
        env_wait(sy + SY_PRE, 1);
        row_store<W>(c, next, cal_section(c, kk + 1));
    }
    write_obs<W>(c, obs_row, c.row[RW_AMB_J], c.row + RW_COUNT, false);
    for (int i = ln(); i < nocc; i += W) c.occ_state[i] = st_new[i];
    for (int z = ln(); z < L->nz; z += W) c.occV[z] = v_new[z];
    STAMP(16);
    env_wait(sy + SY_POST, 1);
    STAMP(17);
    double* hzq = reinterpret_cast<double*>(env + L->lds.hzq);
    zone_means<W>(c, hzq);
    esync();
    const RewardPart part = reward_rest<W>(c, hzq, v_new);
    if (ln() == 0) *reinterpret_cast<RewardPart*>(sy + SY_PART) = part;
    // the observation row's stores are complete before the first wavefront
    // may overwrite the row with an auto-reset observation
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    env_post(sy + SY_HALF, 1);
    STAMP(18);
    // the record's field, mass, VAV and AHU arrays [0, early) are final (the
    // first wavefront changes them after this only when the episode ends,
    // and then stores them again after SY_STORED): stored here, beside its
    // bookkeeping, so the end of the step stores only the rest
    store16<W>(c.rec, env + L->lds.state, 0, L->st.plant & ~15);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): complete before the first wavefront may store them again
    env_post(sy + SY_STORED, 1);
    stamps_flush(P, c);
}

// One workgroup per tile of E envs of one layout, two wavefronts per env:
// wavefronts [0, E) step the envs, wavefronts [E, 2E) are their helpers (the
// helper of env slot s is wavefront E + (s + E - E/2) % E, on another SIMD
// than its env's first wavefront).
template <int W, int KV>
__global__ __launch_bounds__(512) void step_kernel(KParams P0) {
    static_assert(W == 64, "one wavefront per env");
    const KParams P = P0;
    extern __shared__ __align__(16) unsigned char lds[];
    const unsigned long long t_entry = P.phase_ts ? wall_clock64() : 0ull;
    const SBK_C Tile& tl = P.tiles[blockIdx.x];
    const SBK_C DevLayout* L = P.layouts + tl.layout;
    const int E = (int)(blockDim.x >> 7);
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));   // wave-uniform
    const bool helper = wv >= E;
    const int slot = helper ? (wv - E + (E >> 1)) % E : wv;
    const bool active = slot < tl.count;
    const int e = tl.env[slot];
    const EnvDesc ed = tl.desc[slot];
    Ctx c;
    c.L = L;
    c.S = P.scens + ed.scen;
    c.e = e;
    c.helper = helper;
    c.conv = c.S->conv_on != 0;
    c.rec = P.state + ed.state_off;
    unsigned char* env = lds + P.img_lds + slot * tl.lds_bytes;
    int* sy = reinterpret_cast<int*>(env + L->lds.sync);
    c.stamps = reinterpret_cast<unsigned long long*>(env + L->lds.stamps);
    // an inactive slot's region may lie past the workgroup's LDS (a layout's
    // tiles hold only the envs that fit): it touches no LDS but the shared image
    if (active) STAMP(0);
    if (P.phase_ts && ln() == 0 && !helper && active) c.stamps[SBK_STAMP_ENTRY] = t_entry;
    {
        // one burst: the layout image (whole block, every thread), and per env
        // (its two wavefronts) its record image, its scenario image and its
        // action row; the LDS pointers are bound while the first round's loads
        // are in flight
        constexpr int UI = 8, UR = 8, US = 2, UA = 1;   // one round: 64 KB of image, 16 KB of record
        constexpr int ET = 2 * W;                        // threads per env
        const int nthr = (int)blockDim.x, tid = (int)threadIdx.x;
        const int et = (helper ? W : 0) + ln();
        const int img16 = tl.img16;
        const int rec16 = active ? tl.rec16 : 0;
        const int scn16 = active ? ed.scn16 : 0;
        const int act16 = (active && P.mode == KMODE_STEP) ? (4 * SB_ACT) >> 4 : 0;
        const SBK_C uint4* isrc = reinterpret_cast<const SBK_C uint4*>(tl.img_src);
        const SBK_C uint4* ssrc = reinterpret_cast<const SBK_C uint4*>(ed.scen_src);
        const uint4* rsrc = reinterpret_cast<const uint4*>(c.rec);
        const uint4* asrc = reinterpret_cast<const uint4*>(P.actions + (size_t)e * SB_ACT);
        uint4* idst = reinterpret_cast<uint4*>(lds);
        uint4* rdst = reinterpret_cast<uint4*>(env + tl.lds_state);
        uint4* sdst = reinterpret_cast<uint4*>(env + tl.lds_scen);
        uint4* adst = reinterpret_cast<uint4*>(env + tl.lds_act);
        const int rounds = max(max((img16 + UI * nthr - 1) / (UI * nthr), (rec16 + UR * ET - 1) / (UR * ET)),
                               max((scn16 + US * ET - 1) / (US * ET), (act16 + UA * ET - 1) / (UA * ET)));
        {
            uint4 pi[UI], pr[UR], ps[US], pa[UA];
            part_load(pi, isrc, img16, tid, nthr, 0);
            part_load(pr, rsrc, rec16, et, ET, 0);
            part_load(ps, ssrc, scn16, et, ET, 0);
            part_load(pa, asrc, act16, et, ET, 0);
            bind(c, lds, env);
            part_pin(pi);
            part_pin(pr);
            part_pin(ps);
            part_pin(pa);
            part_store(pi, idst, img16, tid, nthr, 0);
            part_store(pr, rdst, rec16, et, ET, 0);
            part_store(ps, sdst, scn16, et, ET, 0);
            part_store(pa, adst, act16, et, ET, 0);
        }
        for (int rd = 1; rd < rounds; rd++) {
            uint4 pi[UI], pr[UR], ps[US], pa[UA];
            part_load(pi, isrc, img16, tid, nthr, rd * UI * nthr);
            part_load(pr, rsrc, rec16, et, ET, rd * UR * ET);
            part_load(ps, ssrc, scn16, et, ET, rd * US * ET);
            part_load(pa, asrc, act16, et, ET, rd * UA * ET);
            part_pin(pi);
            part_pin(pr);
            part_pin(ps);
            part_pin(pa);
            part_store(pi, idst, img16, tid, nthr, rd * UI * nthr);
            part_store(pr, rdst, rec16, et, ET, rd * UR * ET);
            part_store(ps, sdst, scn16, et, ET, rd * US * ET);
            part_store(pa, adst, act16, et, ET, rd * UA * ET);
        }
        if (active && !helper && P.mode == KMODE_STEP) {
            const SBK_C uint4* src = reinterpret_cast<const SBK_C uint4*>(L->pinfo);
            for (int i = ln(); i < L->n_pass; i += W) reinterpret_cast<uint4*>(c.prec)[i] = src[i];
        }
        if (active && !helper && ln() < SY_WORDS) sy[ln()] = 0;
    }
    __syncthreads();   // the only workgroup barrier: the layout image is shared
    if (!active) return;
    const bool reset_mode = P.mode == KMODE_RESET;
    // the step's calendar index and step count, read before either wavefront
    // changes them (the first one advances the index after SY_SENS)
    const int kk0 = c.ip[PI_STEP_INDEX], st0 = c.ip[PI_STEP];
    c.row = cal_section(c, kk0);
    if (helper) {
        if (!reset_mode) helper_step<W, KV>(c, P, sy, env, P.obs + (size_t)e * 1024, kk0, ed.start + st0 + 1);
        return;
    }
    STAMP(1);
    float* obs_row = P.obs + (size_t)e * 1024;
    // the step (KMODE_STEP), then one shared reset path for puf_reset and for
    // the auto-reset at the end of an episode
    int done = 0;
    const int early = L->st.plant & ~15;   // the part of the record stored after the field step
    if (!reset_mode) {
        decode_apply<W>(c);
        STAMP(2);
        step_pre<W>(c, P, sy);
        if (P.air_trace) {
            // the step's air side as the reference core's state holds it (air_g, air_T)
            double* at = P.air_trace + (size_t)e * 2 * P.air_stride;
            for (int col = ln(); col < L->k; col += W) {
                at[col] = c.g[col];
                at[P.air_stride + col] = c.tair[col];
            }
        }
        STAMP(3);
        step_post<W>(c);             // boiler update: reads the pre-step results, not the field
        env_post(sy + SY_PRE, 1);    // the helper's observation reads the state as of here
        STAMP(4);
        field_step<W, KV>(c, P, sy);
        if (c.conv) {
            env_wait(sy + SY_CONV, 1);   // the helper's permutation of the room cells
            conv_apply<W>(c);
        }
        env_post(sy + SY_POST, 1);   // the helper's reward half reads the new field
        STAMP(7);
        zone_means<W>(c, c.zq);
        esync();
        double blower, cooling;
        reward_ahu<W>(c, c.zq, blower, cooling);
        STAMP(8);
        env_wait(sy + SY_HALF, 1);   // the helper's reward half, observation and new occupancy
        STAMP(9);
        const RewardPart part = *reinterpret_cast<const RewardPart*>(sy + SY_PART);
        StepParts sp;
        const double rew = reward_combine(c, blower, cooling, part, sp);
        const float r = (float)rew;
        const int step = c.ip[PI_STEP] + 1;
        // the first episode after puf_vec_create may be cut short (desync); a
        // cut episode is a truncation and stays out of the episode log
        // (complete_port/gpu/smart_buildings.cu:1990-1993, 2043)
        const bool first = c.ip[PI_FIRST_DONE] == 0;
        const bool cut = first && ed.first_steps < ed.max_steps;
        done = step >= (first ? ed.first_steps : ed.max_steps);
        if (ln() == 0) {
            P.rewards[e] = r * P.reward_scale;
            P.terminals[e] = done ? 1.0f : 0.0f;
            c.ip[PI_STEP] = step;
            c.plant[PF_REW_SUM] += rew;
            c.plant[PF_DEV_SUM] += sp.v[3];
            c.ip[PI_STEPS_TOTAL] += 1;
            if (done) {
                c.ip[PI_EPISODES] += 1;
                c.ip[PI_FIRST_DONE] = 1;
            }
        }
        // the episode's running sums in float, as the reference GPU env keeps
        // them (smart_buildings.cu:1965-1971), lane k updating sum k; added to
        // the host Log when a whole episode ends (:2002-2036), so a step reads
        // nothing over the host link
        float* ep = reinterpret_cast<float*>(c.ip + PI_EP);
        {
            const int k = ln();
            float x = r;
#pragma unroll
            for (int q = 0; q < 8; q++) x = k == EP_PART + q ? (float)sp.v[q] : x;
            if (k < EP_COUNT) {
                const float o = ep[k];
                ep[k] = k == EP_WORST ? ((float)sp.v[4] > o ? (float)sp.v[4] : o) : o + x;
            }
        }
        esync();
        if (done) {
            if (P.host_env && !cut) log_episode(P, e, ep, step);
            esync();
            if (ln() < EP_COUNT) ep[ln()] = 0.0f;
        }
        esync();
    }
    if (reset_mode || done) {
        env_reset<W>(c, ed.start, obs_row, reset_mode);
        if (reset_mode && ln() == 0) {
            c.ip[PI_STEP] = 0;
            c.ip[PI_STEPS_TOTAL] = 0;
            c.ip[PI_EPISODES] = 0;
#pragma unroll
            for (int k = 0; k < EP_COUNT; k++) c.ip[PI_EP + k] = 0;
            c.plant[PF_REW_SUM] = 0.0;
            c.plant[PF_DEV_SUM] = 0.0;
        }
    }
    esync();
    STAMP(10);
    // the helper has stored the record's field, mass, VAV and AHU arrays
    // [0, early); an episode that ended rewrote them (the reset), so once the
    // helper's stores are complete they are stored again
    if (!reset_mode && done) env_wait(sy + SY_STORED, 1);
    store16<W>(c.rec, env + L->lds.state, (reset_mode || done) ? 0 : early, L->st.bytes);
    STAMP(11);
    stamps_flush(P, c);
}

// Beta(2,2) action rows (see sbx_gen_actions in sbenv.h): the median of three
// U(0,1) of one Philox4x32-10 block keyed by the seed, counter (env, step, slot, 0).
__device__ __forceinline__ float beta22(uint64_t seed, uint32_t env, uint32_t step, uint32_t slot) {
    const Ctr4 r = philox4x32_10(Ctr4{env, step, slot, 0u}, (uint32_t)seed, (uint32_t)(seed >> 32));
    float a = u24(r.x), b = u24(r.y), d = u24(r.z);
    float lo = a < b ? a : b, hi = a < b ? b : a;
    return d < lo ? lo : (d > hi ? hi : d);
}

__global__ void gen_actions_kernel(float* actions, const int* n_cont, const int* n_disc, int n_envs,
                                   uint64_t seed, uint32_t step) {
#pragma clang fp contract(off)
    const int e = blockIdx.x;
    if (e >= n_envs) return;
    const int nc = n_cont[e], nd = n_disc[e];
    float* row = actions + (size_t)e * SB_ACT;
    for (int i = threadIdx.x; i < SB_ACT; i += blockDim.x) {
        float v = 0.0f;
        if (i < SB_CONT) {
            if (i < nc) v = 2.0f * beta22(seed, (uint32_t)e, step, (uint32_t)i) - 1.0f;
        } else {
            int d = i - SB_CONT;
            if (d < nd) v = beta22(seed, (uint32_t)e, step, (uint32_t)i) > 0.5f ? 1.0f : 0.0f;
        }
        row[i] = v;
    }
}

// puf_live_log's totals: workgroup 0 over every env, out[0] the f64 sum of
// rewards since puf_reset, out[1] env-steps since puf_reset, out[2] episodes
// ended since puf_reset; workgroup 1 + g over scenario g's envs, out[3 + 3g]
// its reward sum, out[4 + 3g] its sum of per-step mean zone deviations, out[5
// + 3g] its env-steps. Each thread sums envs t, t + 256, ... in ascending
// order, then a fixed tree: the result does not depend on timing. Field
// scenarios' envs are added after, by their own kernel.
__global__ __launch_bounds__(256) void live_sums_kernel(const EnvDesc* envs, const DevLayout* layouts,
                                                        const unsigned char* state, int n, double* out) {
    __shared__ double red[3][256];
    const int t = (int)threadIdx.x;
    const int g = (int)blockIdx.x - 1;   // -1: every env
    double a0 = 0.0, a1 = 0.0, a2 = 0.0;
    for (int i = t; i < n; i += 256) {
        const EnvDesc& d = envs[i];
        const DevLayout* L = layouts + d.layout;
        if (L->st.bytes == 0) continue;   // a field scenario's env (its totals are added after)
        if (g >= 0 && d.scen != g) continue;
        const unsigned char* r = state + d.state_off;
        const double* pf = reinterpret_cast<const double*>(r + L->st.plant);
        const int* ip = reinterpret_cast<const int*>(r + L->st.iplant);
        a0 += pf[PF_REW_SUM];
        if (g < 0) {
            a1 += (double)ip[PI_STEPS_TOTAL];
            a2 += (double)ip[PI_EPISODES];
        } else {
            a1 += pf[PF_DEV_SUM];
            a2 += (double)ip[PI_STEPS_TOTAL];
        }
    }
    red[0][t] = a0;
    red[1][t] = a1;
    red[2][t] = a2;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w)
            for (int q = 0; q < 3; q++) red[q][t] += red[q][t + w];
        __syncthreads();
    }
    if (t < 3) out[(g < 0 ? 0 : 3 + 3 * g) + t] = red[t][0];
}

}  // namespace sbk

// ---------------------------------------------------------------- launchers
extern "C" int sbk_launch_live_sums(const sbk::EnvDesc* envs, const sbk::DevLayout* layouts,
                                    const unsigned char* state, int n, int n_scen, double* out, hipStream_t s) {
    hipLaunchKernelGGL(sbk::live_sums_kernel, dim3(1 + n_scen), dim3(256), 0, s, envs, layouts, state, n, out);
    return (int)hipGetLastError();
}

// threads: 128 per env of a tile (two wavefronts; at most 4 envs per workgroup).
extern "C" int sbk_launch_step(const sbk::KParams* p, int n_blocks, int threads, int lds_bytes, int variant,
                               hipStream_t s) {
    using namespace sbk;
    if (threads < 128 || threads > 512 || threads % 128) return (int)hipErrorInvalidValue;
    const dim3 g(n_blocks), b(threads);
    switch (variant) {
    case KV_LU: hipLaunchKernelGGL((step_kernel<64, KV_LU>), g, b, lds_bytes, s, *p); break;
    case KV_POINT: hipLaunchKernelGGL((step_kernel<64, KV_POINT>), g, b, lds_bytes, s, *p); break;
    case KV_BLOCK: hipLaunchKernelGGL((step_kernel<64, KV_BLOCK>), g, b, lds_bytes, s, *p); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

extern "C" int sbk_set_lds_limit(int width, int bytes) {
    using namespace sbk;
    if (width != 64) return (int)hipErrorInvalidValue;
    const void* fns[KV_COUNT] = {(const void*)step_kernel<64, KV_LU>, (const void*)step_kernel<64, KV_POINT>,
                                 (const void*)step_kernel<64, KV_BLOCK>};
    for (const void* f : fns) {
        const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}

extern "C" int sbk_launch_gen_actions(float* actions, const int* n_cont, const int* n_disc, int n_envs,
                                      uint64_t seed, uint32_t step, hipStream_t s) {
    hipLaunchKernelGGL(sbk::gen_actions_kernel, dim3(n_envs), dim3(256), 0, s, actions, n_cont, n_disc, n_envs,
                       seed, step);
    return (int)hipGetLastError();
}
