// Canonical policy interface of the env (env kwargs canonical = 1, residual),
// on the device: the env's own observation stays in an internal row, and two
// small kernels around the step give the policy its canonical view.
//
//   canon_pre_kernel   (before the step) the policy's canonical action row and
//                      the base controller's proposal -> the env's native
//                      action row (residual: base + res_scale p, run bits
//                      (2 base - 1) + res_dscale p > 0; absolute: p, run bits
//                      p > -0.5; p clamped to [-1, 1], non-finite -> 0, times
//                      the comfort guard's trust when it is on), which the step
//                      kernel then decodes as any action row
//                      (complete_port/gpu/sb_gpu_base.inc:371-404 decode_res_k);
//   canon_post_kernel  (after the step or reset) from the env's new observation:
//                      the pid_water base controller's proposal for the next
//                      step and its PID state (zeroed when the env starts an
//                      episode; complete_port/submission/pidw_base.py
//                      PIDWaterResetPolicy, zones of an AHU in observation
//                      order, its float32 / float64 arithmetic op by op), the
//                      comfort guard's trust (sb_gpu_base.inc:230-265), and the
//                      canonical observation into the trainer's row
//                      (sb_gpu_base.inc:287-369).
// One 64-lane workgroup per env: zone slots across lanes, one lane per AHU,
// the building-wide hot-water reset on lane 0, features across lanes; the
// env's proposal and trust are kept in LDS until they are written out.
#include <hip/hip_runtime.h>
#include <math.h>

#include "canon.h"
#include "sbenv_internal.h"

namespace sbk {

// numpy's pairwise sum of n < 128 values (8 accumulators), then / n
template <class T>
__device__ __forceinline__ T np_mean(const T* a, int n) {
#pragma clang fp contract(off)
    T r;
    if (n < 8) {
        r = T(0);
        for (int i = 0; i < n; i++) r = r + a[i];
    } else {
        T q[8];
        for (int j = 0; j < 8; j++) q[j] = a[j];
        int i = 8;
        for (; i < n - (n % 8); i += 8)
            for (int j = 0; j < 8; j++) q[j] = q[j] + a[i + j];
        r = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
        for (; i < n; i++) r = r + a[i];
    }
    return r / (T)n;
}

// pidw_base.py _cyclic_feature_to_index: float32 arctan2 (rounded from
// float64), + 2 pi when negative, floor(period * angle / (2 pi)) in float32
__device__ __forceinline__ int cyclic(float s, float c, int period) {
#pragma clang fp contract(off)
    float ang = (float)atan2((double)s, (double)c);
    if (ang < 0.0f) ang = ang + (float)(2.0 * 3.141592653589793);
    const float v = ((float)period * ang) / (float)(2.0 * 3.141592653589793);
    return (int)floorf(v);
}

__device__ __forceinline__ double clipd(double x, double lo, double hi) { return x < lo ? lo : (x > hi ? hi : x); }

__device__ __forceinline__ float nat(const CanonTab& C, const float* o, int i) {
#pragma clang fp contract(off)
    return i >= 0 ? o[i] * C.fstd[i] + C.fmean[i] : 0.0f;
}

__global__ __launch_bounds__(64) void canon_post_kernel(CanonArgs A) {
#pragma clang fp contract(off)
    const int e = blockIdx.x, lane = (int)threadIdx.x;
    if (e >= A.n) return;
    const CanonTab& C = A.tabs[A.envs[e].layout];
    const float* o = A.raw_obs + (size_t)e * SB_OBS;
    __shared__ float sb[SB_ACT], sw[SB_ACT], sT[SBC_ZS], st[SBC_ZS], sai[2 * SBC_K], swk[SBC_K];
    __shared__ double spid[2 * SBC_K], seff[SBC_K];
    __shared__ int sact[SBC_K], sheat[SBC_K];
    const bool fresh = A.reset || A.terminals[e] == 1.0f;   // a new episode starts here
    for (int i = lane; i < 2 * SBC_K; i += 64) {
        spid[i] = fresh ? 0.0 : A.pid[(size_t)e * 2 * SBC_K + i];
        sai[i] = 0.0f;
    }
    for (int i = lane; i < SB_ACT; i += 64) {
        sb[i] = 0.0f;
        sw[i] = 1.0f;
    }
    __syncthreads();
    const int hour = cyclic(o[C.g[0]], o[C.g[4]], 24);
    const int day = cyclic(o[C.g[8]], o[C.g[12]], 7);
    const bool work = day < 5 && C.morning <= hour && hour < C.evening;
    const double lo = work ? C.comfort_lo : C.eco_lo, hi = work ? C.comfort_hi : C.eco_hi;
    const float lof = (float)lo, hif = (float)hi;
    // zone commands (PIDProportionalReheatPolicy._command_zones) and the
    // guard's trust per zone, one zone slot per lane
    for (int s = lane; s < SBC_ZS; s += 64) {
        if (C.zT[s] < 0) continue;
        const float T = o[C.zT[s]] * C.tstd + C.tmean;
        sT[s] = T;
        float err = 0.0f;
        if (T < lof) err = lof - T;
        else if (T > hif) err = hif - T;
        const float damper = fminf(1.0f, fabsf(err) / 2.0f);
        if (C.zAd[s] >= 0) sb[C.zAd[s]] = 2.0f * damper - 1.0f;
        const float opening = fminf(1.0f, fmaxf(0.0f, err) / 2.0f);
        if (C.zAr[s] >= 0) sb[C.zAr[s]] = 2.0f * opening - 1.0f;
        if (A.guard) {
            const float dev = T < lof ? lof - T : (A.hot && T > hif ? T - hif : 0.0f);
            const float t = fminf(1.0f, fmaxf(0.0f, 1.0f - (dev - A.d0) / A.d1));
            st[s] = t;
            if (C.zAd[s] >= 0) sw[C.zAd[s]] = t;
            if (C.zAr[s] >= 0) sw[C.zAr[s]] = t;
        }
    }
    __syncthreads();
    // one lane per AHU: its PID loop on the mean zone temperature, fan
    // pressure, run command and economiser (PIDWorstZonePolicy.get_action with
    // PIDEconomizerPolicy's average-zone error and recirculation)
    if (lane < C.K) {
        const int k = lane, nz = C.zc[k];
        sact[k] = 0;
        sheat[k] = 0;
        seff[k] = 0.0;
        if (C.aRec[k] >= 0) sb[C.aRec[k]] = 1.0f;
        if (nz > 0) {
            const double avg = (double)np_mean<float>(sT + SBC_ZPA * k, nz);
            sai[2 * k + 1] = (float)avg;
            double error = 0.0;
            if (avg < lo) error = lo - avg;
            else if (avg > hi) error = hi - avg;
            double* ps = spid + 2 * k;
            if (error == 0.0) {
                ps[0] = ps[0] * 0.5;
                ps[1] = 0.0;
                if (C.aT[k] >= 0) sb[C.aT[k]] = -1.0f;
                if (C.aP[k] >= 0) sb[C.aP[k]] = -1.0f;
                if (C.aRun[k] >= 0) sb[C.aRun[k]] = 0.0f;
            } else {
                ps[0] = clipd(ps[0] + error, -10.0, 10.0);
                const double deriv = error - ps[1];
                ps[1] = error;
                const double u = clipd(0.5 * error + 0.02 * ps[0] + 0.1 * deriv, -1.0, 1.0);
                sai[2 * k] = (float)u;
                seff[k] = u;
                sact[k] = 1;
                sheat[k] = error > 0.0;
                const double pressure = clipd(2.0 * fabs(u) - 1.0, -1.0, 1.0);
                if (C.aT[k] >= 0) sb[C.aT[k]] = (float)u;
                if (C.aP[k] >= 0) sb[C.aP[k]] = (float)pressure;
                if (C.aRun[k] >= 0) sb[C.aRun[k]] = 1.0f;
                if (C.aRec[k] >= 0) {
                    double rec = 1.0;
                    const int oat = C.aObs[k][0];
                    if (!(u >= 0.0) && oat >= 0) {
                        const double outside = (double)o[oat], inside = avg;
                        if (isfinite(outside) && !(outside >= inside)) {
                            double pa = (pressure + 1.0) * 0.5 * 2000.0;
                            pa = pa > 200.0 ? pa : 200.0;
                            if (!(inside - outside <= pa * 0.00322)) {
                                double target = 285.0 + (u + 1.0) * 0.5 * 20.0;
                                target = target > lo ? target : lo;
                                if (!(inside <= target)) {
                                    const double f = (inside - target) / (inside - outside);
                                    rec = 2.0 * clipd(1.0 - f, 0.0, 1.0) - 1.0;
                                }
                            }
                        }
                    }
                    sb[C.aRec[k]] = (float)rec;
                }
            }
        }
        if (A.guard) {
            float wk = 1.0f;
            for (int j = 0; j < nz; j++) wk = fminf(wk, st[SBC_ZPA * k + j]);
            if (C.aT[k] >= 0) sw[C.aT[k]] = wk;
            if (C.aP[k] >= 0) sw[C.aP[k]] = wk;
            if (C.aRec[k] >= 0) sw[C.aRec[k]] = wk;
            if (C.aRun[k] >= 0) sw[C.aRun[k]] = wk;
            swk[k] = wk;
        }
    }
    __syncthreads();
    // the hot-water loop (PIDPolicy's water actions, then PIDWaterResetPolicy's
    // reset: the greater of the mean zone shortfall over 4 K and the 0.25
    // quantile of the AHUs' heating effort)
    if (lane == 0) {
        int any_heat = 0, any_act = 0;
        for (int k = 0; k < C.K; k++) {
            any_heat |= sheat[k];
            any_act |= sact[k];
        }
        if (C.hW >= 0) sb[C.hW] = any_heat ? 1.0f : -1.0f;
        if (C.hDPa >= 0) sb[C.hDPa] = any_act ? 1.0f : -1.0f;
        if (C.hRun >= 0) sb[C.hRun] = any_act ? 1.0f : 0.0f;
        if (C.hW >= 0 && sb[C.hW] > 0.0f) {
            // a shortfall of 0 is a Python 0.0 in the reference's list, which
            // makes numpy's mean float64; with none the mean is float32
            float s32[SBC_ZS];
            double s64[SBC_ZS];
            int ns = 0;
            bool all_pos = true;
            for (int k = 0; k < C.K; k++)
                for (int j = 0; j < C.zc[k]; j++) {
                    const float d = lof - sT[SBC_ZPA * k + j];
                    s32[ns] = d;
                    s64[ns] = d > 0.0f ? (double)d : 0.0;
                    all_pos = all_pos && d > 0.0f;
                    ns++;
                }
            double shortfall = 0.0;
            if (ns > 0) shortfall = all_pos ? (double)np_mean<float>(s32, ns) : np_mean<double>(s64, ns);
            const double demand = shortfall / 4.0;
            double sat = 0.0;
            double h[SBC_K];
            int ne = 0;
            for (int k = 0; k < C.K; k++)
                if (sact[k]) h[ne++] = seff[k] > 0.0 ? seff[k] : 0.0;
            if (ne > 0) {
                for (int i = 1; i < ne; i++) {
                    const double x = h[i];
                    int j = i - 1;
                    while (j >= 0 && h[j] > x) {
                        h[j + 1] = h[j];
                        j--;
                    }
                    h[j + 1] = x;
                }
                // numpy quantile, method linear: virtual index (n - 1) q, numpy's _lerp
                const double vi = (double)(ne - 1) * 0.25;
                int i0 = (int)floor(vi), i1 = i0 + 1;
                if (vi >= (double)(ne - 1)) i0 = i1 = ne - 1;
                const double t = vi - floor(vi);
                const double diff = h[i1] - h[i0];
                sat = t >= 0.5 ? h[i1] - diff * (1.0 - t) : h[i0] + diff * t;
            }
            const double m = demand > sat ? demand : sat;
            sb[C.hW] = (float)(2.0 * clipd(m + 0.0, 0.0, 1.0) - 1.0);
        }
        if (A.guard) {
            float wb = 1.0f;
            for (int k = 0; k < C.K; k++) wb = fminf(wb, swk[k]);
            if (C.hW >= 0) sw[C.hW] = wb;
            if (C.hDPa >= 0) sw[C.hDPa] = wb;
            if (C.hRun >= 0) sw[C.hRun] = wb;
        }
    }
    __syncthreads();
    for (int i = lane; i < SB_ACT; i += 64) {
        A.base[(size_t)e * SB_ACT + i] = sb[i];
        A.trust[(size_t)e * SB_ACT + i] = sw[i];
    }
    for (int i = lane; i < 2 * SBC_K; i += 64) {
        A.pid[(size_t)e * 2 * SBC_K + i] = spid[i];
        A.ainfo[(size_t)e * 2 * SBC_K + i] = sai[i];
    }
    // the canonical observation (residual_policy.py _features)
    float* out = A.obs + (size_t)e * SB_OBS;
    for (int f = lane; f < SBC_OBS; f += 64) {
        float v = 0.0f;
        if (f < SBC_OA) {
            const int s = f / SBC_FZ, c = f % SBC_FZ;
            if (C.zT[s] >= 0) {
                const float T = nat(C, o, C.zT[s]), Hs = nat(C, o, C.zH[s]), Cs = nat(C, o, C.zC[s]);
                switch (c) {
                case 0: v = 1.0f; break;
                case 1: v = (T - 295.0f) / 5.0f; break;
                case 2: v = (T - Hs) / 2.0f; break;
                case 3: v = (Cs - T) / 2.0f; break;
                case 4: v = (Hs - 294.0f) / 3.0f; break;
                case 5: v = C.zD[s] >= 0 ? 2.0f * nat(C, o, C.zD[s]) - 1.0f : 0.0f; break;
                case 6: v = C.zR[s] >= 0 ? 2.0f * nat(C, o, C.zR[s]) - 1.0f : 0.0f; break;
                case 7: v = C.zAd[s] >= 0 ? sb[C.zAd[s]] : 0.0f; break;
                default: v = C.zAr[s] >= 0 ? sb[C.zAr[s]] : 0.0f; break;
                }
            }
        } else if (f < SBC_OH) {
            const int k = (f - SBC_OA) / SBC_FA, c = (f - SBC_OA) % SBC_FA;
            if (k < C.K) {
                const int* q = C.aObs[k];
                switch (c) {
                case 0: v = 1.0f; break;
                case 1: v = (nat(C, o, q[0]) - 283.0f) / 15.0f; break;
                case 2: v = nat(C, o, q[1]) / 1000.0f; break;
                case 3: v = nat(C, o, q[2]) / 10.0f; break;
                case 4: v = nat(C, o, q[3]) / 10.0f; break;
                case 5: v = q[4] >= 0 ? (nat(C, o, q[4]) - 295.0f) / 5.0f : 0.0f; break;
                case 6: v = 2.0f * nat(C, o, q[5]) - 1.0f; break;
                case 7: v = nat(C, o, q[6]) / 10.0f; break;
                case 8: v = 2.0f * nat(C, o, q[7]) - 1.0f; break;
                case 9: v = C.aT[k] >= 0 ? sb[C.aT[k]] : 0.0f; break;
                case 10: v = C.aP[k] >= 0 ? sb[C.aP[k]] : 0.0f; break;
                case 11: v = C.aRec[k] >= 0 ? sb[C.aRec[k]] : 0.0f; break;
                case 12: v = C.aRun[k] >= 0 ? 2.0f * sb[C.aRun[k]] - 1.0f : 0.0f; break;
                case 13: v = C.zc[k] > 0 ? (sai[2 * k + 1] - 295.0f) / 5.0f : 0.0f; break;
                case 14: v = (float)(spid[2 * k] / 10.0); break;
                default: v = sai[2 * k]; break;
                }
            }
        } else if (f < SBC_OG) {
            const int c = f - SBC_OH;
            const int* q = C.hObs;
            switch (c) {
            case 0: v = 1.0f; break;
            case 1: v = (nat(C, o, q[0]) - 330.0f) / 20.0f; break;
            case 2: v = (nat(C, o, q[1]) - 330.0f) / 20.0f; break;
            case 3: v = nat(C, o, q[2]) / 10.0f; break;
            case 4: v = nat(C, o, q[3]) / 10.0f; break;
            case 5: v = 2.0f * nat(C, o, q[4]) - 1.0f; break;
            case 6: v = nat(C, o, q[5]) / 10.0f; break;
            case 7: v = C.hW >= 0 ? sb[C.hW] : 0.0f; break;
            case 8: v = C.hDPa >= 0 ? sb[C.hDPa] : 0.0f; break;
            default: v = C.hRun >= 0 ? 2.0f * sb[C.hRun] - 1.0f : 0.0f; break;
            }
        } else {
            const int i = C.g[f - SBC_OG];
            v = i >= 0 ? o[i] : 0.0f;
        }
        out[f] = v;
    }
    if (A.reset)
        for (int f = SBC_OBS + lane; f < SB_OBS; f += 64) out[f] = 0.0f;
}

__global__ __launch_bounds__(64) void canon_pre_kernel(CanonArgs A) {
#pragma clang fp contract(off)
    const int e = blockIdx.x, lane = (int)threadIdx.x;
    if (e >= A.n) return;
    const CanonTab& C = A.tabs[A.envs[e].layout];
    const float* prow = A.actions + (size_t)e * SB_ACT;
    float* row = A.native + (size_t)e * SB_ACT;
    for (int col = lane; col < SB_ACT; col += 64) {
        const int i = C.act_of_col[col];
        float v = 0.0f;
        if (i >= 0) {
            const int sl = C.slot_of_action[i];
            float p = 0.0f;
            if (sl >= 0) {
                p = prow[sl];
                p = isfinite(p) ? fminf(1.0f, fmaxf(-1.0f, p)) : 0.0f;
                if (A.guard) p = p * A.trust[(size_t)e * SB_ACT + i];
            }
            const float b = A.base[(size_t)e * SB_ACT + i];
            if (C.act_disc[i]) {
                const bool on = A.resid ? (2.0f * b - 1.0f) + A.dscale * p > 0.0f : p > -0.5f;
                v = on ? 1.0f : 0.0f;
            } else {
                const float m = A.resid ? b + A.scale * p : p;
                v = fminf(1.0f, fmaxf(-1.0f, m));
            }
        }
        row[col] = v;
    }
}

}  // namespace sbk

extern "C" int sbk_launch_canon(const sbk::CanonArgs* a, int post, hipStream_t s) {
    if (a->n <= 0) return (int)hipErrorInvalidValue;
    if (post) hipLaunchKernelGGL(sbk::canon_post_kernel, dim3(a->n), dim3(64), 0, s, *a);
    else hipLaunchKernelGGL(sbk::canon_pre_kernel, dim3(a->n), dim3(64), 0, s, *a);
    return (int)hipGetLastError();
}
