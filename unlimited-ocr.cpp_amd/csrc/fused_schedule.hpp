// Static schedule of the fused decode kernel (decode_fused.hip), shared by the
// kernel and by the host-side check uocr_hip_fused_schedule_check (capi.hip),
// which replays it as a wait/publish simulation on the CPU.
//
// Workgroups [0, T) are the routers (one progress step), [T, P) the PW = P - T
// gate/up workers. Gate/up item i (group i / RBG of the G groups, routed ones
// first) -> worker T + i % PW as its step i / PW + 1; it waits for nothing.
// Down items j = (live group j / RBD, block j % RBD) go to "slots" in the
// order the workgroups behind them are expected to be free -- workers with one
// gate/up item fewer, workers that are first on their CU (issue priority goes
// to the older workgroup), the routers, then the rest; a second round of down
// items lands on the first slots -- and wait for the group's gate/up items.
// The combine of column block rb runs on slot (ndn_total + rb) % P after that
// slot's own down items and waits for the routers and the block's down items.
#pragma once

namespace uocr_hip {

struct FusedSchedule {
    int T, P, PW, RBG, RBD, ngu_total, ndn_total, rem, n1, nA;

    __host__ __device__ FusedSchedule(int T_, int P_, int n_groups, int rbg, int rbd, int n_live)
        : T(T_), P(P_), PW(P_ - T_), RBG(rbg), RBD(rbd), ngu_total(n_groups * rbg), ndn_total(n_live * rbd) {
        rem = ngu_total % PW;  // workers T .. T+rem-1 hold one gate/up item more
        n1 = PW - rem;
        nA = rem < P / 2 - T ? rem : P / 2 - T;
        if (nA < 0) nA = 0;
    }
    // gate/up items of workgroup w
    __host__ __device__ int n_gu_of(int w) const {
        if (w < T) return 0;
        const int q = w - T;
        return ngu_total > q ? (ngu_total - 1 - q) / PW + 1 : 0;
    }
    // publisher of gate/up item i and the step it publishes the item as
    __host__ __device__ void gu_step(int i, int& owner, int& step) const {
        owner = T + i % PW;
        step = i / PW + 1;
    }
    __host__ __device__ int slot_wg(int sl) const {
        if (sl < n1) return T + rem + sl;
        sl -= n1;
        if (sl < nA) return T + sl;
        sl -= nA;
        if (sl < T) return sl;
        return T + nA + (sl - T);
    }
    // inverse of slot_wg
    __host__ __device__ int slot_of(int b) const {
        if (b < T) return n1 + nA + b;
        const int q = b - T;
        return q >= rem ? q - rem : (q < nA ? n1 + q : n1 + T + q);
    }
    // publisher of down item j and the step it publishes the item as
    __host__ __device__ void dn_step(int j, int& owner, int& step) const {
        owner = slot_wg(j % P);
        step = (owner < T ? 1 : 0) + n_gu_of(owner) + j / P + 1;
    }
    __host__ __device__ int combine_slot(int rb) const { return (ndn_total + rb) % P; }
};

}  // namespace uocr_hip
