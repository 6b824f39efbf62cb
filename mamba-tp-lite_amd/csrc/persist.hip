// The whole fused decode step of a small model (MambaLM.step, reference
// model.py:343-353 over MambaBlock.step 308-311 and MambaMixer.step 249-294)
// as one persistent launch, fp32, batch 1, followed by the norm_f + tied
// lm_head GEMV of mtl_decode_norm_gemv.
//
// Why one launch.  At the mamba-130m shape a layer of the multi-kernel step
// (decode_in, decode_ssm, decode_gemv) costs ~12 us against ~2 us of weight
// bytes: each of its three dependent kernels pays a graph node (~1.65 us) and
// a cold memory round trip.  Here G workgroups (one per CU) stay resident for
// all layers and meet at three exchanges per layer instead:
//   EA  the x_proj split-K partials of every workgroup's channel block
//   EB  the SSM output y of every channel
//   EC  the new residual row of every out_proj row
// An exchange is a set of 8-byte slots, each holding one fp32 value and the
// tag of the exchange that wrote it, stored with agent-scope (L2-bypassing,
// cross-XCD coherent) relaxed stores and polled with agent-scope relaxed
// loads.  A value is ready when its own tag matches, so no flag, counter,
// atomic read-modify-write or fence is needed (a fence would write back the
// L2).  Every exchange is a full rendezvous: a workgroup can only produce the
// next exchange's values after it has consumed the previous one, so each
// slot array is reused every layer; tags differ per exchange and per launch
// (an epoch kept in the workspace advances by 3 L per launch).
//
// Roles inside a 512-thread workgroup.  Wavefronts 0-1 only poll exchanges:
// vector memory loads complete in order, so a wavefront with weight loads in
// flight could not see an exchange arrive before its weights did.
// Wavefronts 2-7 compute, and after consuming one layer's operands they
// issue the next layer's into the same registers (the SSM operands, in_proj
// rows and conv operands after the SSM phase, the out_proj rows after
// out_proj), so the weight stream of layer l + 1 overlaps the exchanges of
// layer l: each group of loads is issued right after the compute
// wavefronts' store into EB or EC, while the exchange wavefronts wait on it,
// and between any load and its use fewer than 63 younger vector memory
// instructions are issued (the vmcnt field a wait can name).  EA, whose
// slots are many (G J), is polled by all eight wavefronts; by then the
// compute wavefronts' loads were issued a phase or more earlier.  The two
// roles meet at six workgroup barriers per layer.
//
// Ownership.  Workgroup g owns channels [g cb, (g + 1) cb) -- their in_proj x
// and z rows, conv history, x_proj partial, SSM state -- and out_proj rows
// [g rb, (g + 1) rb).  The states are updated in place by their owner only.
//
// Sums run in fixed orders (x_proj partials in workgroup order), so a step is
// deterministic and a graph replay equals eager execution bit for bit.
//
// Waits are bounded: a wait that exceeds kSpinLimit polls writes a code
// naming this launch into the error word of the workspace, stops waiting for
// later exchanges and lets the launch finish; the final residual, and so
// the logits, of that launch are then NaN.  A workgroup of such a launch
// that started after workgroup 0 advanced the epoch tags its slots for the
// next launch, so the caller zero-fills the workspace again before reusing
// it (the host API says so).  All G
// workgroups must be resident at once: the host keeps G at most the CU count
// and checks the occupancy.

#include "common.h"

namespace mtl {
namespace {

constexpr int kPT = 512;                 // threads per workgroup
constexpr int kPWaves = kPT / 64;        // 8
constexpr int kXW = 2;                   // exchange wavefronts (0, 1)
constexpr int kCW = kPWaves - kXW;       // compute wavefronts (2..7)
constexpr int kXT = kXW * 64;            // 128 exchange threads
constexpr int kCT = kCW * 64;            // 384 compute threads
constexpr int kMaxQ = 16;                // workgroup ranges the partial sums are split into
constexpr int kMaxJ = 128;               // x_proj rows (dt_rank + 2 d_state) at most
constexpr int kMaxKc = 4;                // d_conv at most
constexpr uint32_t kSpinLimit = 1u << 15;
constexpr int kMaxLayers = 64;           // cache pointers travel in the kernel arguments
constexpr int kEaRows = 256 + 32;        // EA rows: 256 workgroups + the rows a lane may read past G

struct PArgs {
    const mtl_decode_layer* layers;      // device copy, [L]: weights (its cache fields are not read)
    float* conv_state[kMaxLayers];       // this call's cache, [b, D, K - 1] per layer
    float* ssm_state[kMaxLayers];        // [b, D, N] per layer
    const int64_t* ids;                  // [1]
    const float* emb;                    // [V, M]
    float* x_out;                        // [M] residual after the last layer
    uint64_t* ea;                        // [kEaRows, J]: slot (g, j) at g J + j (rows g >= G read, never waited on)
    uint64_t* eb;                        // [2048] (D used)
    uint64_t* ec;                        // [1024] (M used)
    uint32_t* ctl;                       // [0] epoch, [1] error word
    int V, L, M, D, N, R, K, J, G, cb, rb, Q, per, xg;
};

__device__ __forceinline__ uint64_t ld_slot(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_slot(uint64_t* p, uint32_t tag, float v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool slot_ready(uint64_t s, uint32_t tag) { return (uint32_t)(s >> 32) == tag; }
__device__ __forceinline__ float slot_value(uint64_t s) { return __uint_as_float((uint32_t)s); }
// tags are odd, so the zero-filled workspace never matches one
__device__ __forceinline__ uint32_t tag_of(uint32_t base, int e) { return 2u * (base + (uint32_t)e) + 1u; }
// the error word a timed-out wait leaves: names the launch (odd, never 0)
__device__ __forceinline__ uint32_t fail_of(uint32_t base) { return 2u * base + 1u; }

__device__ __forceinline__ float4 ntload4p(const float* p) {
    typedef float F4 __attribute__((ext_vector_type(4)));
    const F4 v = __builtin_nontemporal_load(reinterpret_cast<const F4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float dot4p(const float4 w, const float4 x, float acc) {
    return fmaf(w.x, x.x, fmaf(w.y, x.y, fmaf(w.z, x.z, fmaf(w.w, x.w, acc))));
}

// Polls the NS slots at byte offsets off + u stride from `base` until the
// first n of them carry `tag`, leaving them in v[].  The address is stepped
// opaquely, so the slot addresses are formed at the poll, one at a time,
// not hoisted out of the layer loop and kept live across it.  On a spin-limit
// overrun the error word is set to this launch's fail_code and *failed is
// raised (later waits are skipped).
template <int NS>
__device__ __forceinline__ void poll_slots(const uint64_t* base, uint32_t off, uint32_t stride, int n, uint32_t tag,
                                           uint64_t* v, uint32_t* err, uint32_t fail_code, bool* failed) {
    // one running address, stepped opaquely: NS addresses are never held at once
    const char* q = reinterpret_cast<const char*>(base) + off;
#pragma unroll
    for (int u = 0; u < NS; ++u) {
        v[u] = ld_slot(reinterpret_cast<const uint64_t*>(q));
        q += stride;
        asm volatile("" : "+v"(q));
    }
    if (*failed) return;
    for (uint32_t spin = 0;; ++spin) {
        bool all = true;
#pragma unroll
        for (int u = 0; u < NS; ++u) all = all && (u >= n || slot_ready(v[u], tag));
        if (all) return;
        if (spin >= kSpinLimit) {
            __hip_atomic_store(err, fail_code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *failed = true;
            return;
        }
        q = reinterpret_cast<const char*>(base) + off;
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            if (u < n && !slot_ready(v[u], tag)) v[u] = ld_slot(reinterpret_cast<const uint64_t*>(q));
            q += stride;
            asm volatile("" : "+v"(q));
        }
    }
}

// PLM / PLD: float4 runs per lane of a d_model / d_inner row (M <= 256 PLM,
// D <= 256 PLD); RQ: dt_proj columns per SSM lane (R <= 16 RQ); RI / RO:
// in_proj / out_proj rows per compute wavefront, so a workgroup holds at
// most kCW RI / 2 channels and kCW RO out_proj rows; XP: x_proj partial
// slots per lane at most (a.per <= XP); WXC: channels per x_proj lane
// (the block's channels split over a.xg groups of lanes per output).
template <int PLM, int PLD, int RQ, int RI, int RO, int XP, int WXC>
__global__ void __launch_bounds__(kPT) decode_persist_kernel(const PArgs a) {
    constexpr int CBX = kCW * RI / 2;                  // channels per workgroup at most
    static_assert(CBX * 16 <= kCT, "one 16-lane SSM row per channel");
    __shared__ __align__(16) float s_r[PLM * 256];     // residual entering the current layer
    __shared__ __align__(16) float s_y[PLD * 256];     // y of every channel
    __shared__ float s_pre[2 * CBX];                   // in_proj outputs: x rows, then z rows
    __shared__ float s_xc[CBX];                        // SiLU(conv) of the channel block
    __shared__ float s_gz[CBX];                        // SiLU(z) of the channel block
    __shared__ float s_q[kMaxQ][kMaxJ];                // x_dbl range sums
    __shared__ float s_xp[kCT];                        // x_proj partials of the channel groups
    __shared__ uint32_t s_base;

    const int tid = threadIdx.x, lane = tid & 63;
    // wavefront-uniform, and known to be so: the role branch below is then a
    // scalar branch, and each role keeps only its own registers live
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = blockIdx.x;
    const int M = a.M, D = a.D, N = a.N, R = a.R, K = a.K, J = a.J, L = a.L, G = a.G;
    const int M4 = M >> 2, D4 = D >> 2;
    const int cb = a.cb, c0 = g * cb, nch = max(0, min(cb, D - c0));
    const int m0 = g * a.rb, nrow = max(0, min(a.rb, M - m0));
    uint32_t* err = a.ctl + 1;
    bool failed = false;

    // EA lanes (every thread): output j = ep of x_proj, workgroups
    // [eq per, eq per + ea_n).  Each workgroup's J partials are one
    // contiguous row written by that workgroup alone (a j-major layout, whose
    // cache lines 16 writers share while 128 workgroups poll them, measured
    // an EA wait of 15 us against 2.5 us).
    const int Q = a.Q, per = a.per;
    const int ep = tid % J, eq = tid / J;
    const bool ea_lane = tid < J * Q;                        // J Q <= kPT
    const int ea_n = ea_lane ? max(0, min(per, G - eq * per)) : 0;
    const uint32_t ea_off = (uint32_t)(min(eq * per, G) * J + ep) * 8u;
    auto poll_ea = [&](int l) __attribute__((always_inline)) {
        uint64_t v[XP];
        poll_slots<XP>(a.ea, ea_off, 8u * (uint32_t)J, ea_n, tag_of(s_base, 3 * l), v, err, fail_of(s_base), &failed);
        float sum = 0.f;
#pragma unroll
        for (int u = 0; u < XP; ++u) sum += u < ea_n ? slot_value(v[u]) : 0.f;
        if (ea_lane) s_q[eq][ep] = sum;
    };

    if (tid == 0) s_base = __hip_atomic_load(a.ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    if (wave < kXW) {
        // ===================================================== exchange wavefronts
        const int x = tid;                                   // 0..127
        {   // the embedding row of the token (an id outside [0, V) reads row 0 and yields NaN)
            const int64_t id = a.ids[0];
            const bool ok = id >= 0 && id < a.V;
            const float* row = a.emb + (ok ? id : 0) * (int64_t)M;
            for (int e = x; e < M; e += kXT) s_r[e] = ok ? row[e] : __builtin_nanf("");
        }
        __syncthreads();                                     // s_r, s_base
        const uint32_t base = s_base;
        for (int l = 0; l < L; ++l) {
            __syncthreads();                                 // s1: in_proj rows done
            __syncthreads();                                 // s2: conv done
            __syncthreads();                                 // s2b: x_proj group partials
            poll_ea(l);
            __syncthreads();                                 // s3: x_dbl range sums
            {   // EB: y of every channel, slots x + 128 u (D <= 256 PLD)
                uint64_t v[2 * PLD];
                const int n = x < D ? (D - x + kXT - 1) / kXT : 0;
                poll_slots<2 * PLD>(a.eb, 8u * (uint32_t)x, 8u * kXT, n, tag_of(base, 3 * l + 1), v, err, fail_of(base),
                                    &failed);
#pragma unroll
                for (int u = 0; u < 2 * PLD; ++u)
                    if (u < n) s_y[x + u * kXT] = slot_value(v[u]);
            }
            __syncthreads();                                 // s4: y
            {   // EC: the new residual, slots x + 128 u (M <= 256 PLM), written
                // into s_r only once every slot (this workgroup's own rows
                // included) has arrived: the compute wavefronts read their
                // rows of the old residual before storing
                uint64_t v[2 * PLM];
                const int n = x < M ? (M - x + kXT - 1) / kXT : 0;
                poll_slots<2 * PLM>(a.ec, 8u * (uint32_t)x, 8u * kXT, n, tag_of(base, 3 * l + 2), v, err, fail_of(base),
                                    &failed);
#pragma unroll
                for (int u = 0; u < 2 * PLM; ++u)
                    if (u < n) s_r[x + u * kXT] = slot_value(v[u]);
            }
            __syncthreads();                                 // s5: residual of the next layer
        }
        if (g == 0) {
            const bool bad = failed || __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == fail_of(base);
            for (int e = x; e < M; e += kXT) a.x_out[e] = bad ? __builtin_nanf("") : s_r[e];
            if (x == 0) __hip_atomic_store(a.ctl, base + 3u * (uint32_t)L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }

    // ========================================================= compute wavefronts
    const int ct = tid - kXT;                                // 0..383
    const int wc = wave - kXW;                               // 0..5
    // in_proj rows of this wavefront: local row li = wc + kCW i; li < cb is
    // the x row of channel c0 + li, cb <= li < 2 cb the z row of c0 + li - cb
    auto in_row = [&](int i) __attribute__((always_inline)) {
        const int li = wc + kCW * i;
        const int ch = li < cb ? li : li - cb;
        const bool ok = li < 2 * cb && ch < nch;
        return min((li < cb ? 0 : D) + c0 + (ok ? ch : 0), 2 * D - 1);
    };
    auto in_ok = [&](int i) __attribute__((always_inline)) {
        const int li = wc + kCW * i;
        return li < 2 * cb && (li < cb ? li : li - cb) < nch;
    };
    auto out_row = [&](int i) __attribute__((always_inline)) { return min(m0 + min(wc + kCW * i, max(nrow - 1, 0)), M - 1); };
    // conv lanes: channel ct of the block; SSM lanes: channel ct / 16, state ct % 16
    const int cv_cc = min(c0 + min(ct, max(nch - 1, 0)), D - 1);     // clamped: a block may hold no channel
    const bool cv_ok = ct < nch;
    const int ss_c = ct >> 4, ss_n = ct & 15;
    const bool ss_row = ss_c < nch;                          // whole 16-lane rows
    const int ss_cc = min(c0 + min(ss_c, max(nch - 1, 0)), D - 1);
    const int ss_nn = min(ss_n, N - 1);
    // x_proj lanes: output xp_j, channels [xp_g WXC, (xp_g + 1) WXC) of the block
    const int xg = a.xg;
    const bool xp_ok = ct < J * xg;
    const int xp_j = ct % J, xp_g = min(ct / J, xg - 1);

    // per-layer operands, loaded one phase after their use for the next layer
    float4 w_in[RI][PLM], nw[PLM], w_out[RO][PLD];
    float b_in[RI], b_out[RO];
    float cst[kMaxKc - 1], cwt[kMaxKc], cbias;
    float wx[WXC];
    float wdt[RQ], alog, bdt, Dc, hst;
    // The loads below run unconditionally, for layer l when live and at one
    // cached line of the last layer otherwise (values unused): a reload under
    // a branch would keep the consumed layer's registers alive across the
    // exchanges that follow.
    // Each helper forms its per-lane offsets from an opaque copy of the lane
    // index, so the compiler does not precompute every (row, run) address
    // once and hold them all in registers across the layer loop.
    auto load_in = [&](int l, bool live) __attribute__((always_inline)) {
        const float* W = a.layers[l].W_in;
        const float* bi = a.layers[l].b_in;
        const int lm = live ? 1 : 0;
        int ol = lane;
        asm volatile("" : "+v"(ol));
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            const int row = in_row(i) * lm;
#pragma unroll
            for (int p = 0; p < PLM; ++p)
                w_in[i][p] = ntload4p(W + (int64_t)row * M + 4 * min(p * 64 + ol, M4 - 1) * lm);
            b_in[i] = bi ? bi[row] : 0.f;
        }
        const float* nwp = a.layers[l].norm_w;
#pragma unroll
        for (int p = 0; p < PLM; ++p) nw[p] = *reinterpret_cast<const float4*>(nwp + 4 * min(p * 64 + ol, M4 - 1) * lm);
    };
    auto load_conv = [&](int l) __attribute__((always_inline)) {
        int cc = cv_cc, xj = xp_j, xc0 = xp_g * WXC;
        asm volatile("" : "+v"(cc), "+v"(xj), "+v"(xc0));
        const float* st = a.conv_state[l] + (int64_t)cc * (K - 1);
        const float* cw = a.layers[l].conv_w + (int64_t)cc * K;
        const float* cbp = a.layers[l].conv_b;
#pragma unroll
        for (int k = 0; k < kMaxKc - 1; ++k) cst[k] = st[min(k, K - 2)];
#pragma unroll
        for (int k = 0; k < kMaxKc; ++k) cwt[k] = cw[min(k, K - 1)];
        cbias = cbp ? cbp[cc] : 0.f;
        const float* wxt = a.layers[l].W_xT;
#pragma unroll
        for (int c = 0; c < WXC; ++c)
            wx[c] = wxt[(int64_t)min(c0 + min(xc0 + c, max(nch - 1, 0)), D - 1) * J + xj];
    };
    auto load_ssm = [&](int l) __attribute__((always_inline)) {
        int sc = ss_cc, sn = ss_n;
        asm volatile("" : "+v"(sc), "+v"(sn));
        const float* W = a.layers[l].W_dt;
#pragma unroll
        for (int q = 0; q < RQ; ++q) wdt[q] = W[(int64_t)sc * R + min(sn + 16 * q, R - 1)];
        alog = a.layers[l].A_log[(int64_t)sc * N + min(sn, N - 1)];
        bdt = a.layers[l].dt_bias[sc];
        const float* dv = a.layers[l].Dv;
        Dc = dv ? dv[sc] : 0.f;
        hst = a.ssm_state[l][(int64_t)sc * N + min(sn, N - 1)];
    };
    auto load_out = [&](int l, bool live) __attribute__((always_inline)) {
        const float* W = a.layers[l].W_out;
        const float* bo = a.layers[l].b_out;
        const int lm = live ? 1 : 0;
        int ol = lane;
        asm volatile("" : "+v"(ol));
#pragma unroll
        for (int i = 0; i < RO; ++i) {
            const int row = out_row(i) * lm;
#pragma unroll
            for (int p = 0; p < PLD; ++p)
                w_out[i][p] = ntload4p(W + (int64_t)row * D + 4 * min(p * 64 + ol, D4 - 1) * lm);
            b_out[i] = bo ? bo[row] : 0.f;
        }
    };
    load_in(0, true);
    load_conv(0);
    load_ssm(0);
    load_out(0, true);
    __syncthreads();                                         // s_r, s_base
    const uint32_t base = s_base;
    const float4* r4 = reinterpret_cast<const float4*>(s_r);
    const float4* y4 = reinterpret_cast<const float4*>(s_y);

    for (int l = 0; l < L; ++l) {
        const bool more = l + 1 < L;
        // ---- A: RMSNorm + in_proj rows (the rms scale applied to the dots)
        {
            float4 xw[PLM];
            float ss = 0.f;
#pragma unroll
            for (int p = 0; p < PLM; ++p) {
                const bool ok = p * 64 + lane < M4;
                const float4 xv = r4[min(p * 64 + lane, M4 - 1)];
                ss = ok ? fmaf(xv.x, xv.x, fmaf(xv.y, xv.y, fmaf(xv.z, xv.z, fmaf(xv.w, xv.w, ss)))) : ss;
                xw[p] = make_float4(nw[p].x * xv.x, nw[p].y * xv.y, nw[p].z * xv.z, nw[p].w * xv.w);
            }
            ss = group_sum<64>(ss);
            const float rs = rsqrtf(ss / (float)M + a.layers[l].eps);
#pragma unroll
            for (int i = 0; i < RI; ++i) {
                float acc = 0.f;
#pragma unroll
                for (int p = 0; p < PLM; ++p) {
                    const float t = dot4p(w_in[i][p], xw[p], acc);
                    acc = p * 64 + lane < M4 ? t : acc;
                }
                acc = group_sum<64>(acc);
                if (lane == 0 && in_ok(i)) s_pre[wc + kCW * i] = fmaf(acc, rs, b_in[i]);
            }
        }
        __syncthreads();                                     // s1
        // ---- conv step (history shifted in place) + SiLU; SiLU(z)
        if (cv_ok) {
            const float xin = s_pre[ct];
            float cacc = 0.f;
#pragma unroll
            for (int k = 0; k < kMaxKc - 1; ++k)
                if (k < K - 1) cacc = fmaf(cst[k], cwt[k], cacc);
#pragma unroll
            for (int k = 0; k < kMaxKc; ++k)
                if (k == K - 1) cacc = fmaf(xin, cwt[k], cacc);
            cacc += cbias;
            float* st = a.conv_state[l] + (int64_t)(c0 + ct) * (K - 1);
#pragma unroll
            for (int k = 0; k < kMaxKc - 2; ++k)
                if (k < K - 2) st[k] = cst[k + 1];
            st[K - 2] = xin;
            s_xc[ct] = silu_f(cacc);
            s_gz[ct] = silu_f(s_pre[cb + ct]);
        }
        __syncthreads();                                     // s2
        // ---- x_proj partial of the block: channel groups, then their sum in
        //      group order -> EA; every thread then polls EA
        if (xp_ok) {
            float xacc = 0.f;
#pragma unroll
            for (int c = 0; c < WXC; ++c) {
                const int ch = xp_g * WXC + c;
                xacc = ch < nch ? fmaf(wx[c], s_xc[min(ch, CBX - 1)], xacc) : xacc;
            }
            s_xp[ct] = xacc;
        }
        __syncthreads();                                     // s2b
        if (ct < J) {
            float xsum = s_xp[ct];
            for (int q = 1; q < xg; ++q) xsum += s_xp[q * J + ct];
            st_slot(a.ea + (int64_t)g * J + ct, tag_of(base, 3 * l), xsum);
        }
        poll_ea(l);
        __syncthreads();                                     // s3: x_dbl range sums in s_q
        const int ln = more ? l + 1 : l;
        // ---- SSM: dt_proj + softplus, state update in place, y -> EB
        if (ss_row) {
            auto xd = [&](int j) __attribute__((always_inline)) {
                float s = s_q[0][j];
                for (int q = 1; q < Q; ++q) s += s_q[q][j];
                return s;
            };
            float dacc = 0.f;
#pragma unroll
            for (int q = 0; q < RQ; ++q) {
                const int jj = ss_n + 16 * q;
                const float t = fmaf(wdt[q], xd(min(jj, R - 1)), dacc);
                dacc = jj < R ? t : dacc;
            }
            dacc = group_sum<16>(dacc);
            const float dt = softplus_f(dacc + bdt);
            const float xv = s_xc[ss_c];
            float yv = 0.f;
            if (ss_n < N) {
                const float av = -expf(alog);
                const float dA = __builtin_amdgcn_exp2f(dt * (av * kLog2e));
                const float hv = fmaf(hst, dA, (dt * xd(R + ss_n)) * xv);
                a.ssm_state[l][(int64_t)(c0 + ss_c) * N + ss_n] = hv;
                yv = hv * xd(R + N + ss_n);
            }
            yv = group_sum<16>(yv);
            if (ss_n == 0) st_slot(a.eb + c0 + ss_c, tag_of(base, 3 * l + 1), (yv + xv * Dc) * s_gz[ss_c]);
        }
        // the next layer's SSM operands, in_proj rows and conv operands
        // stream while the exchange wavefronts wait on EB
        load_ssm(ln);
        load_in(ln, more);
        load_conv(ln);
        __syncthreads();                                     // s4: y in s_y
        // ---- out_proj rows + the residual add -> EC
        {
            float acc[RO];
#pragma unroll
            for (int i = 0; i < RO; ++i) acc[i] = 0.f;
#pragma unroll
            for (int p = 0; p < PLD; ++p) {
                const bool ok = p * 64 + lane < D4;
                const float4 yv = y4[min(p * 64 + lane, D4 - 1)];
#pragma unroll
                for (int i = 0; i < RO; ++i) {
                    const float t = dot4p(w_out[i][p], yv, acc[i]);
                    acc[i] = ok ? t : acc[i];
                }
            }
#pragma unroll
            for (int i = 0; i < RO; ++i) {
                acc[i] = group_sum<64>(acc[i]);
                if (lane == 0 && wc + kCW * i < nrow) {
                    const int m = out_row(i);
                    st_slot(a.ec + m, tag_of(base, 3 * l + 2), s_r[m] + (acc[i] + b_out[i]));
                }
            }
        }
        load_out(ln, more);                                  // streams while EC is awaited
        __syncthreads();                                     // s5: the next layer's residual in s_r
    }
}

// Register blockings instantiated: (RI, RO) in_proj and out_proj rows per
// compute wavefront and XP partial slots per lane.  persist_config picks
// the first whose grid fits: fewer workgroups exchange fewer partials (G^2 J
// slots per layer), more stream the weights faster (one workgroup reads
// 48-56 GB/s from HBM); at the 130m shape 64 workgroups measured faster
// than 128 (449 against 489 us per token).
struct Blocking {
    int RI, RO, XP;
};
constexpr Blocking kBlockings[] = {{8, 2, 16}, {4, 1, 24}};
constexpr int kWXC = 8;                  // channels per x_proj lane at most

struct PersistConfig {
    int G, RI, RO, XP, Q, per, xg;
};

// The grid of a blocking: enough workgroups that each holds at most
// kCW RI / 2 channels and kCW RO out_proj rows; the EA lanes of Q ranges
// must cover the G partials with at most XP slots each, and the channel
// groups of the x_proj lanes at most kWXC channels each.
bool persist_config(int M, int D, int J, int cus, int only, PersistConfig* out) {
    for (int bi = 0; bi < (int)(sizeof(kBlockings) / sizeof(kBlockings[0])); ++bi) {
        if (only && only != bi + 1) continue;
        const Blocking& bl = kBlockings[bi];
        const int cbx = kCW * bl.RI / 2, rbx = kCW * bl.RO;
        const int G = std::max({(D + cbx - 1) / cbx, (M + rbx - 1) / rbx, 1});
        if (G > cus) continue;
        const int Q = std::max(1, std::min(kMaxQ, kPT / J));
        const int per = (G + Q - 1) / Q;
        if (per > bl.XP) continue;
        const int cb = (D + G - 1) / G;
        const int xg = std::max(1, std::min(kCT / J, cb));
        if ((cb + xg - 1) / xg > kWXC) continue;
        *out = PersistConfig{G, bl.RI, bl.RO, bl.XP, Q, per, xg};
        return true;
    }
    return false;
}

}  // namespace
}  // namespace mtl

extern "C" size_t mtl_decode_persist_workspace_bytes(int32_t d_model, int32_t d_inner, int32_t d_state,
                                                     int32_t dt_rank) {
    (void)d_model;
    (void)d_inner;
    const size_t J = (size_t)dt_rank + 2 * (size_t)d_state;
    // control words; EA for up to 256 workgroups and 32 rows of padding (a
    // lane reads XP <= 24 rows from its range start, which is at most G); EB
    // and EC at the largest d_inner and d_model taken (reads stay in bounds)
    return 256 + 8 * ((size_t)mtl::kEaRows * J + 2048 + 1024);
}

extern "C" int32_t mtl_decode_persist_grid(int32_t d_model, int32_t d_inner, int32_t d_state, int32_t dt_rank,
                                           int32_t d_conv, int32_t n_layers, int32_t blocking) {
    using namespace mtl;
    const int32_t J = dt_rank + 2 * d_state;
    if (d_model < 4 || d_model % 4 || d_model > 1024 || d_inner < 4 || d_inner % 4 || d_inner > 2 * d_model ||
        d_state < 1 || d_state > 16 || dt_rank < 1 || dt_rank > 64 || J > kMaxJ || d_conv < 2 || d_conv > kMaxKc ||
        n_layers < 1 || n_layers > kMaxLayers || blocking < 0 || blocking > 2)
        return 0;
    PersistConfig cfg;
    return persist_config(d_model, d_inner, J, 256, blocking, &cfg) ? cfg.G : 0;
}

extern "C" int mtl_decode_step_persist(const mtl_decode_step_args* a, const mtl_decode_layer* layers,
                                       const mtl_decode_layer* layers_dev, void* workspace, size_t workspace_bytes,
                                       int32_t blocking, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(a && layers && layers_dev && workspace, "null args, layers, layers_dev or workspace");
    const int32_t b = a->batch, M = a->d_model, D = a->d_inner, N = a->d_state, R = a->dt_rank, K = a->d_conv;
    const int32_t J = R + 2 * N;
    MTL_REQUIRE(b == 1, "batch must be 1");
    MTL_REQUIRE(a->n_layers >= 1 && a->n_layers <= kMaxLayers && a->vocab >= 1,
                "n_layers must be in [1, 64] and vocab >= 1");
    MTL_REQUIRE(blocking >= 0 && blocking <= 2, "blocking must be 0 (automatic), 1 or 2");
    MTL_REQUIRE(M >= 4 && M % 4 == 0 && M <= 1024, "d_model must be a multiple of 4, at most 1024");
    MTL_REQUIRE(D >= 4 && D % 4 == 0 && D <= 2 * M, "d_inner must be a multiple of 4, at most 2 d_model");
    MTL_REQUIRE(N >= 1 && N <= 16 && R >= 1 && R <= 64 && J <= kMaxJ,
                "d_state must be in [1, 16], dt_rank in [1, 64] and dt_rank + 2 d_state at most 128");
    MTL_REQUIRE(K >= 2 && K <= kMaxKc, "d_conv must be 2, 3 or 4");
    MTL_REQUIRE(a->ids && a->emb && a->norm_f && a->logits && a->x0, "null ids, emb, norm_f, logits or x0");
    MTL_REQUIRE(workspace_bytes >= mtl_decode_persist_workspace_bytes(M, D, N, R), "workspace too small");
    MTL_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-byte aligned");
    auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    MTL_REQUIRE(al16(a->x0) && al16(a->emb), "x0 and emb must be 16-byte aligned");
    MTL_REQUIRE(a->x0 != a->logits, "logits must not alias x0");
    for (int32_t i = 0; i < a->n_layers; ++i) {
        const mtl_decode_layer& L = layers[i];
        const std::string at = "layer " + std::to_string(i) + ": ";
        MTL_REQUIRE(L.norm_w && L.W_in && L.conv_w && L.W_xT && L.W_dt && L.dt_bias && L.A_log && L.W_out &&
                    L.conv_state && L.ssm_state, at + "null required pointer (W_xT included)");
        MTL_REQUIRE(al16(L.W_in) && al16(L.W_out) && al16(L.norm_w), at + "W_in, W_out and norm_w must be 16-byte aligned");
    }
    int dev = 0, cus = 0;
    if (hipStreamGetDevice(as_stream(stream), &dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
        set_error("mtl_decode_step_persist: cannot query the device");
        return MTL_EHIP;
    }
    PersistConfig cfg;
    MTL_REQUIRE(persist_config(M, D, J, std::min(cus, 256), blocking, &cfg),
                "no register blocking fits this shape on this device");
    const int PLM = round_runs((M / 4 + 63) / 64);
    const int RQ = (R + 15) / 16;

    uint8_t* ws = static_cast<uint8_t*>(workspace);
    PArgs p;
    p.layers = layers_dev; p.ids = a->ids; p.emb = a->emb; p.x_out = a->x0;
    for (int i = 0; i < kMaxLayers; ++i) {
        p.conv_state[i] = i < a->n_layers ? layers[i].conv_state : nullptr;
        p.ssm_state[i] = i < a->n_layers ? layers[i].ssm_state : nullptr;
    }
    p.ctl = reinterpret_cast<uint32_t*>(ws);
    p.ea = reinterpret_cast<uint64_t*>(ws + 256);
    p.eb = p.ea + (size_t)kEaRows * J;
    p.ec = p.eb + 2048;
    p.V = a->vocab; p.L = a->n_layers; p.M = M; p.D = D; p.N = N; p.R = R; p.K = K; p.J = J; p.G = cfg.G;
    p.cb = (D + cfg.G - 1) / cfg.G; p.rb = (M + cfg.G - 1) / cfg.G; p.Q = cfg.Q; p.per = cfg.per; p.xg = cfg.xg;
    hipStream_t st = as_stream(stream);

    // every workgroup must be resident at once (each waits on all the others)
    auto launch = [&](auto kern) -> int {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kPT, 0) != hipSuccess || per_cu < 1) {
            set_error("mtl_decode_step_persist: the kernel does not fit a CU");
            return MTL_EHIP;
        }
        hipLaunchKernelGGL(kern, dim3((unsigned)cfg.G), dim3(kPT), 0, st, p);
        return check_launch("decode_persist");
    };
    // d_inner <= 2 d_model: PLD = 2 PLM covers it
    int rc = MTL_EINVAL;
#define MTL_PERSIST_RQ(PM, RIV, ROV, XPV)                                                        \
    switch (RQ) {                                                                               \
        case 1: rc = launch(decode_persist_kernel<PM, 2 * PM, 1, RIV, ROV, XPV, kWXC>); break;   \
        case 2: rc = launch(decode_persist_kernel<PM, 2 * PM, 2, RIV, ROV, XPV, kWXC>); break;   \
        case 3: rc = launch(decode_persist_kernel<PM, 2 * PM, 3, RIV, ROV, XPV, kWXC>); break;   \
        default: rc = launch(decode_persist_kernel<PM, 2 * PM, 4, RIV, ROV, XPV, kWXC>); break;  \
    }
#define MTL_PERSIST_PLM(RIV, ROV, XPV)                                                           \
    switch (PLM) {                                                                              \
        case 1: MTL_PERSIST_RQ(1, RIV, ROV, XPV) break;                                         \
        case 2: MTL_PERSIST_RQ(2, RIV, ROV, XPV) break;                                         \
        case 3: MTL_PERSIST_RQ(3, RIV, ROV, XPV) break;                                         \
        default: MTL_PERSIST_RQ(4, RIV, ROV, XPV) break;                                        \
    }
    if (cfg.RI == 8) {
        MTL_PERSIST_PLM(8, 2, 16)
    } else {
        MTL_PERSIST_PLM(4, 1, 24)
    }
#undef MTL_PERSIST_PLM
#undef MTL_PERSIST_RQ
    if (rc) return rc;
    return mtl_decode_norm_gemv(a->x0, a->norm_f, a->eps_f, a->emb, nullptr, a->logits, 1, a->vocab, M, stream);
}
