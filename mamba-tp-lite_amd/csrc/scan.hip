// Fused selective-scan prefill for gfx950.
//
// Replaces the materialize-then-loop scan of mamba-tp-lite model.py:216-238
// (and its TP-shard twin tp_model.py:110-129): dt bias + softplus, dA =
// exp(dt*A), dBx = dt*B*x, the sequential recurrence, y = C.h, the D skip and
// the silu(z) gate, plus the final state (model.py:241) -- in one pass over
// HBM with nothing of shape [b, D, l, N] ever materialized.
//
// Work decomposition (one workgroup = 64 channels of one batch row):
//   * 4 wavefronts; wavefront w carries states [w*SPW, (w+1)*SPW) of all 64
//     channels in registers (lane = channel).  B_t[n] and C_t[n] are then
//     uniform across the wavefront and are read as LDS broadcasts; no
//     cross-lane traffic happens inside the time loop.
//   * The sequence is walked in tiles of TT timesteps.  All 256 threads load
//     the tile of u / delta / z coalesced (layout-specialized), compute
//     dt = softplus(delta + bias), dt*u and silu(z) ONCE per (channel, t)
//     and stage dt, dt*u in LDS.  The next tile's raw loads are issued
//     before the scan of the current one (register double buffering).
//   * Each wavefront writes its partial y_t (sum over its states) to LDS;
//     the loader threads add the 4 partials in a fixed order (deterministic),
//     apply (y + D*u) * silu(z) and store y coalesced.
// Per (channel, t, state) the inner loop costs one v_exp_f32 and four VALU
// ops (mul, mul, fma, fma).  dt is staged in log2 units (dt * log2 e, which
// softplus_l2_f returns directly), so exp(dt * A) is exp2(dt_l2 * A); the
// injection dt * u * B then takes its ln 2 from B, scaled where B is staged.

#include <type_traits>

#include "common.h"

namespace mtl {
namespace {

struct ScanArgs {
    const void* u; const void* delta; const void* z; const void* B; const void* C; void* y;
    const float* A; const float* Dv; const float* dbias; const float* h0; float* h_out;
    int64_t u_sb, u_sd, u_sl;
    int64_t d_sb, d_sd, d_sl;
    int64_t z_sb, z_sd, z_sl;
    int64_t B_sb, B_sn, B_sl;
    int64_t C_sb, C_sn, C_sl;
    int64_t y_sb, y_sd, y_sl;
    int L, D, N;
    int softplus, a_is_log;
};

// E contiguous activations <-> floats (E a multiple of 4; 16-byte (fp32) or
// 8-byte (bf16) aligned when VEC).
template <typename T, int E, bool VEC>
__device__ __forceinline__ void load_run(const T* p, float* v) {
    if constexpr (VEC && sizeof(T) == 4) {
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            const float4 x = reinterpret_cast<const float4*>(p)[q];
            v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
        }
    } else if constexpr (VEC && sizeof(T) == 2) {
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            const uint2 x = reinterpret_cast<const uint2*>(p)[q];
            v[4 * q] = __uint_as_float(x.x << 16); v[4 * q + 1] = __uint_as_float(x.x & 0xffff0000u);
            v[4 * q + 2] = __uint_as_float(x.y << 16); v[4 * q + 3] = __uint_as_float(x.y & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int j = 0; j < E; ++j) v[j] = Act<T>::load(p + j);
    }
}
template <typename T, int E, bool VEC>
__device__ __forceinline__ void store_run(T* p, const float* v) {
    if constexpr (VEC && sizeof(T) == 4) {
#pragma unroll
        for (int q = 0; q < E / 4; ++q)
            reinterpret_cast<float4*>(p)[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    } else if constexpr (VEC && sizeof(T) == 2) {
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            uint2 x;
            x.x = f32x2_to_bf16x2(v[4 * q], v[4 * q + 1]);
            x.y = f32x2_to_bf16x2(v[4 * q + 2], v[4 * q + 3]);
            reinterpret_cast<uint2*>(p)[q] = x;
        }
    } else {
#pragma unroll
        for (int j = 0; j < E; ++j) Act<T>::store(p + j, v[j]);
    }
}

template <bool B> using Full = std::integral_constant<bool, B>;

// p + off bytes, for a wavefront-uniform p and a 32-bit per-lane offset: the
// load then takes the base from SGPRs and only the offset from a VGPR, with
// no 64-bit address arithmetic on the VALU.
template <typename T>
__device__ __forceinline__ T* at_bytes(T* p, uint32_t off) {
    using C = typename std::conditional<std::is_const<T>::value, const char, char>::type;
    return reinterpret_cast<T*>(reinterpret_cast<C*>(p) + off);
}

// Token-major rows through buffer instructions: a resource (SGPRs) based at
// the first row of a thread's run of steps, the lane's channel as the VGPR
// byte offset and the step within the run as the SGPR offset -- no VALU
// address arithmetic at all.  The resource's range covers exactly the run's
// rows, so an access outside them reads 0 / is dropped instead of faulting.
constexpr int kBufWord3 = 0x00020000;   // raw (untyped) 32-bit data format
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kBufWord3);
}
template <typename T> struct BufAct;
template <> struct BufAct<float> {
    __device__ __forceinline__ static float load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)vo, (int)so, 0));
    }
    __device__ __forceinline__ static void store(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, float v) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)vo, (int)so, 0);
    }
};
template <> struct BufAct<uint16_t> {
    __device__ __forceinline__ static float load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
        return bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, (int)vo, (int)so, 0));
    }
    __device__ __forceinline__ static void store(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, float v) {
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), r, (int)vo, (int)so, 0);
    }
};

// 4 consecutive activations of a channel-major row through a buffer
// resource: a wavefront-uniform SGPR offset (the tile's first step) plus the
// lane's loop-invariant VGPR offset, so no VALU address arithmetic per tile.
typedef unsigned int U4v __attribute__((ext_vector_type(4)));
typedef unsigned int U2v __attribute__((ext_vector_type(2)));
template <typename T> struct Buf4;
template <> struct Buf4<float> {
    __device__ __forceinline__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, float* v) {
        const U4v x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, (int)so, 0);
        v[0] = __uint_as_float(x.x); v[1] = __uint_as_float(x.y);
        v[2] = __uint_as_float(x.z); v[3] = __uint_as_float(x.w);
    }
    __device__ __forceinline__ static void store(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, const float* v) {
        const U4v x = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
        __builtin_amdgcn_raw_buffer_store_b128(x, r, (int)vo, (int)so, 0);
    }
};
template <> struct Buf4<uint16_t> {
    __device__ __forceinline__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, float* v) {
        const U2v x = __builtin_amdgcn_raw_buffer_load_b64(r, (int)vo, (int)so, 0);
        v[0] = __uint_as_float(x.x << 16); v[1] = __uint_as_float(x.x & 0xffff0000u);
        v[2] = __uint_as_float(x.y << 16); v[3] = __uint_as_float(x.y & 0xffff0000u);
    }
    __device__ __forceinline__ static void store(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, const float* v) {
        const U2v x = {f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])};
        __builtin_amdgcn_raw_buffer_store_b64(x, r, (int)vo, (int)so, 0);
    }
};

// NW wavefronts per workgroup = NW state groups of SPW states over the same
// 64 channels.  CM: channel-major [b,D,l] rows (l-stride 1); otherwise
// token-major (D-stride 1).  VEC: CM rows are aligned for vector access and
// each tensor's batch row spans under 2^31 bytes (buffer offsets).
//
// A load tile is KC sub-tiles of TT steps: channel-major rows are read KC*TT
// steps at a time (a whole 128-byte line per row for fp32 when KC*TT = 32,
// both halves requested back to back) and y is written the same way, while
// the scan works through LDS one TT-step sub-tile at a time.  Token-major
// reads are full lines at any tile length, so there KC = 1.
// Channel-major tiles hold twice the raw registers (3 waves per SIMD);
// token-major ones fit 128 VGPRs, so 4 workgroups share a CU.
// GEN: softplus and the z gate follow the runtime flags; without it both are
// on (the mixer's case), and the staging has no per-element selects for them.
template <typename T, int NW, int SPW, int TT, bool CM, bool VEC, bool GEN>
__global__ void __launch_bounds__(NW * 64, CM ? 3 : 4) scan_fwd_kernel(const ScanArgs a) {
    constexpr int NT = NW * 64;
    constexpr int E = TT * 64 / NT;            // consecutive steps one thread stages per sub-tile
    constexpr int KC = CM ? 2 : 1;             // sub-tiles per load tile
    constexpr int LT = KC * TT;                // steps per load tile
    constexpr int NP = NW * SPW;               // padded state count
    constexpr int BCE = (NP * LT + NT - 1) / NT;
    constexpr int TS = TT + 4;                 // [c][t] LDS row stride: 16B aligned, b128 conflict-free
    constexpr int BS = NP + 4;                 // padded B/C rows: staging writes spread over banks
    static_assert(E % 4 == 0, "tile shape");

    __shared__ __align__(16) float s_dt[64][TS];
    __shared__ __align__(16) float s_dx[64][TS];
    __shared__ __align__(16) float s_y[NW][64][TS];
    __shared__ __align__(16) float s_B[LT][BS];
    __shared__ __align__(16) float s_C[LT][BS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    // XCD-aware tile order: workgroups are dealt to the 8 XCDs round robin,
    // so workgroup w takes tile (w % 8) * (tiles / 8) + w / 8.  Each XCD then
    // works through whole batch rows, and a row's B/C tiles are fetched from
    // HBM into one L2 instead of all eight (reads 1.08 -> 1.005x the
    // algorithmic bytes at [32,1536,1024])
    int wlin = blockIdx.y * gridDim.x + blockIdx.x;
    const int wtot = gridDim.x * gridDim.y;
    if (wtot % 8 == 0) wlin = (wlin % 8) * (wtot / 8) + wlin / 8;
    const int b = wlin / gridDim.x;
    const int c0 = (wlin - b * gridDim.x) * 64;
    const int L = a.L, D = a.D, N = a.N;

    // staging ownership: channel oc and, in sub-tile kc, steps
    // [kc*TT + ot, kc*TT + ot + E).  Token-major puts 64 channels on the 64
    // lanes.  Channel-major gives each wavefront 64/NW channels x all NW row
    // segments (the same addresses per load instruction as any other split),
    // with the channel fastest across lanes so 8 adjacent lanes hit distinct
    // LDS bank groups.
    constexpr int CPW = 64 / NW;               // channels per wavefront (CM)
    const int oc = CM ? wave * CPW + lane % CPW : lane;
    const int ot = CM ? (lane / CPW) * E : wave * E;
    const bool c_ok = c0 + oc < D;
    const int cl = c_ok ? c0 + oc : D - 1;     // loads of a tail channel block read a valid row

    const T* __restrict__ up = static_cast<const T*>(a.u) + b * a.u_sb + (int64_t)cl * (CM ? a.u_sd : 1);
    const T* __restrict__ dp = static_cast<const T*>(a.delta) + b * a.d_sb + (int64_t)cl * (CM ? a.d_sd : 1);
    const bool has_z = !GEN || a.z != nullptr;
    const bool do_softplus = !GEN || a.softplus;
    // without a gate z aliases u: its loads stay unconditional (a branch
    // around them would merge registers through copies that wait for loads)
    const T* __restrict__ zp = has_z ? static_cast<const T*>(a.z) + b * a.z_sb + (int64_t)cl * (CM ? a.z_sd : 1)
                                     : up;
    const int64_t z_sl = has_z ? a.z_sl : a.u_sl;
    T* __restrict__ yp = static_cast<T*>(a.y) + b * a.y_sb + (int64_t)cl * (CM ? a.y_sd : 1);
    const T* __restrict__ Bp = static_cast<const T*>(a.B) + b * a.B_sb;
    const T* __restrict__ Cp = static_cast<const T*>(a.C) + b * a.C_sb;
    const bool bc_t_fast = a.B_sl == 1;
    // token-major rows: the step's row start is uniform per wavefront (SGPRs),
    // the lane's channel is a byte offset into it
    const T* __restrict__ ub = static_cast<const T*>(a.u) + b * a.u_sb;
    const T* __restrict__ db = static_cast<const T*>(a.delta) + b * a.d_sb;
    const T* __restrict__ zb = has_z ? static_cast<const T*>(a.z) + b * a.z_sb : ub;
    T* __restrict__ yb = static_cast<T*>(a.y) + b * a.y_sb;
    const uint32_t ch_bytes = (uint32_t)cl * (uint32_t)sizeof(T);
    const int ot_u = CM ? 0 : __builtin_amdgcn_readfirstlane(ot);   // token-major: ot = wave * E
    // step strides and the byte span of E consecutive rows (host-checked < 2^31)
    const uint32_t sl_bytes_u = (uint32_t)(a.u_sl * (int64_t)sizeof(T));
    const uint32_t sl_bytes_d = (uint32_t)(a.d_sl * (int64_t)sizeof(T));
    const uint32_t sl_bytes_z = (uint32_t)(z_sl * (int64_t)sizeof(T));
    const uint32_t sl_bytes_y = (uint32_t)(a.y_sl * (int64_t)sizeof(T));
    const uint32_t row_bytes = (uint32_t)D * (uint32_t)sizeof(T);
    const uint32_t run_bytes_u = (E - 1) * sl_bytes_u + row_bytes;
    const uint32_t run_bytes_d = (E - 1) * sl_bytes_d + row_bytes;
    const uint32_t run_bytes_z = (E - 1) * sl_bytes_z + row_bytes;
    const uint32_t run_bytes_y = (E - 1) * sl_bytes_y + row_bytes;

    // channel-major full tiles: resources over one batch row of each tensor,
    // the lane's channel row and staging offset as a loop-invariant VGPR offset
    auto cm_rsrc = [&](const void* p, int64_t sb, int64_t sd) {
        return row_rsrc(static_cast<const T*>(p) + b * sb, (uint32_t)(((int64_t)(D - 1) * sd + L) * (int64_t)sizeof(T)));
    };
    const auto ru_cm = cm_rsrc(a.u, a.u_sb, a.u_sd);
    const auto rd_cm = cm_rsrc(a.delta, a.d_sb, a.d_sd);
    const auto rz_cm = has_z ? cm_rsrc(a.z, a.z_sb, a.z_sd) : ru_cm;
    const auto ry_cm = cm_rsrc(a.y, a.y_sb, a.y_sd);
    const uint32_t vo_u = (uint32_t)(((int64_t)cl * a.u_sd + ot) * (int64_t)sizeof(T));
    const uint32_t vo_d = (uint32_t)(((int64_t)cl * a.d_sd + ot) * (int64_t)sizeof(T));
    const uint32_t vo_z = has_z ? (uint32_t)(((int64_t)cl * a.z_sd + ot) * (int64_t)sizeof(T)) : vo_u;
    const uint32_t vo_y = (uint32_t)(((int64_t)cl * a.y_sd + ot) * (int64_t)sizeof(T));

    const float bias_c = (a.dbias ? a.dbias[cl] : 0.f) * kLog2e;   // log2 units, as dt
    const float D_c = a.Dv ? a.Dv[cl] : 0.f;

    // scan registers: states [wave*SPW, wave*SPW + SPW) of channel c0 + lane
    const bool lane_ok = c0 + lane < D;
    float h[SPW], a2[SPW];
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        const int n = wave * SPW + k;
        const bool ok = lane_ok && n < N;
        float av = ok ? a.A[(int64_t)(c0 + lane) * N + n] : 0.f;
        if (ok && a.a_is_log) av = -expf(av);
        a2[k] = av;
        h[k] = (ok && a.h0) ? a.h0[((int64_t)b * D + c0 + lane) * N + n] : 0.f;
    }

    // The lambdas below are forced inline: an outlined one takes the state
    // arrays it captures through scratch memory (seen at 2 wavefronts x 8
    // states: 6x slower).
    // raw load-tile registers: two sets, so the next load tile is in flight
    // while the current one is scanned
    struct Raw { float u[KC][E], d[KC][E], z[KC][E], B[BCE], C[BCE]; };
    Raw r0;
    [[maybe_unused]] Raw r1;
    float du[E], gz[E];
    float yout[KC][E];

    // B/C staging slots of this thread (loop invariant): element e = tid + NT*k
    // of the [LT x NP] tile.  Loads always read a valid address (state and
    // time clamped); out-of-range slots are zeroed when staged.  No select
    // consumes a loaded register before the stage, so the prefetch stays in
    // flight across the scan (a select right after a load would force a wait
    // for every outstanding load).
    int bc_off[BCE], bc_t[BCE], bc_slot[BCE];
    uint32_t b_bytes[BCE], c_bytes[BCE];     // element (state, step) of a full tile, from the tile's row
    bool bc_ok[BCE];
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
        const int e = tid + NT * k;
        const int n = bc_t_fast ? e / LT : e % NP;
        const int t = bc_t_fast ? e % LT : e / NP;
        bc_ok[k] = e < NP * LT && n < N;
        bc_t[k] = min(t, LT - 1);
        bc_off[k] = min(n, N - 1);
        bc_slot[k] = (e < NP * LT) ? bc_t[k] * BS + n : -1;
        b_bytes[k] = (uint32_t)((bc_off[k] * a.B_sn + bc_t[k] * a.B_sl) * (int64_t)sizeof(T));
        c_bytes[k] = (uint32_t)((bc_off[k] * a.C_sn + bc_t[k] * a.C_sl) * (int64_t)sizeof(T));
    }

    // the raw u / delta / z of sub-tile kc of the load tile at tb
    auto load_sub = [&](Raw& r, int tb, int kc, auto full) __attribute__((always_inline)) {
        constexpr bool F = decltype(full)::value;
        {
            const int t0 = tb + kc * TT + ot;
            if constexpr (CM && VEC) {
                // Full tiles put the tile's first step in the SGPR offset.  A
                // partial tile reads past L into the next row, or past the end
                // of the resource on the last row: its step goes into the VGPR
                // offset, which the buffer range check covers (reads past the
                // resource return 0); staging masks those steps either way.
                const uint32_t st = (uint32_t)(tb + kc * TT) * (uint32_t)sizeof(T);
                const uint32_t so = F ? st : 0u, vs = F ? 0u : st;
#pragma unroll
                for (int q = 0; q < E / 4; ++q) {
                    Buf4<T>::load(ru_cm, vo_u + vs + q * 4 * sizeof(T), so, &r.u[kc][4 * q]);
                    Buf4<T>::load(rd_cm, vo_d + vs + q * 4 * sizeof(T), so, &r.d[kc][4 * q]);
                    Buf4<T>::load(rz_cm, vo_z + vs + q * 4 * sizeof(T), so, &r.z[kc][4 * q]);
                }
            } else if constexpr (CM && F) {
                load_run<T, E, VEC>(up + t0, r.u[kc]);
                load_run<T, E, VEC>(dp + t0, r.d[kc]);
                load_run<T, E, VEC>(zp + t0, r.z[kc]);
            } else if constexpr (CM) {
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    const int t = F ? t0 + j : min(t0 + j, L - 1);
                    r.u[kc][j] = Act<T>::load(up + t);
                    r.d[kc][j] = Act<T>::load(dp + t);
                    r.z[kc][j] = Act<T>::load(zp + t);
                }
            } else {
                // token-major: one buffer resource per tensor over the E rows of
                // this thread's run; step j is an SGPR offset
                const int tw = tb + kc * TT + ot_u;
                const int t0c = F ? tw : min(tw, L - 1);
                const auto ru = row_rsrc(ub + (int64_t)t0c * a.u_sl, run_bytes_u);
                const auto rd = row_rsrc(db + (int64_t)t0c * a.d_sl, run_bytes_d);
                const auto rz = row_rsrc(zb + (int64_t)t0c * z_sl, run_bytes_z);
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    const uint32_t dj = (uint32_t)((F ? tw + j : min(tw + j, L - 1)) - t0c);
                    r.u[kc][j] = BufAct<T>::load(ru, ch_bytes, dj * sl_bytes_u);
                    r.d[kc][j] = BufAct<T>::load(rd, ch_bytes, dj * sl_bytes_d);
                    r.z[kc][j] = BufAct<T>::load(rz, ch_bytes, dj * sl_bytes_z);
                }
            }
        }
    };
    // the raw B / C of the load tile at tb
    auto load_bc = [&](Raw& r, int tb, auto full) __attribute__((always_inline)) {
        constexpr bool F = decltype(full)::value;
        if constexpr (F) {
            const T* Bt = Bp + (int64_t)tb * a.B_sl;
            const T* Ct = Cp + (int64_t)tb * a.C_sl;
#pragma unroll
            for (int k = 0; k < BCE; ++k) {
                r.B[k] = Act<T>::load(at_bytes(Bt, b_bytes[k]));
                r.C[k] = Act<T>::load(at_bytes(Ct, c_bytes[k]));
            }
        } else {
#pragma unroll
            for (int k = 0; k < BCE; ++k) {
                const int t = min(tb + bc_t[k], L - 1);
                r.B[k] = Act<T>::load(Bp + bc_off[k] * a.B_sn + (int64_t)t * a.B_sl);
                r.C[k] = Act<T>::load(Cp + bc_off[k] * a.C_sn + (int64_t)t * a.C_sl);
            }
        }
    };
    auto load_tile = [&](Raw& r, int tb, auto full) __attribute__((always_inline)) {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) load_sub(r, tb, kc, full);
        load_bc(r, tb, full);
    };

    // stage sub-tile kc of the load tile at tb (B/C of the whole load tile
    // are staged with sub-tile 0)
    auto stage_tile = [&](const Raw& r, int tb, int kc, auto full) __attribute__((always_inline)) {
        constexpr bool F = decltype(full)::value;
        float vdt[E], vdx[E];
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const bool ok = F || tb + kc * TT + ot + j < L;
            float dt = fmaf(r.d[kc][j], kLog2e, bias_c);   // (delta + bias) * log2 e
            if (do_softplus) dt = softplus_l2_f(dt);
            const float uv = ok ? r.u[kc][j] : 0.f;
            dt = ok ? dt : 0.f;                 // zero steps leave the state untouched past the end
            vdt[j] = dt;
            vdx[j] = dt * uv;
            du[j] = uv;                         // D * u is folded into the output fma
            gz[j] = has_z ? silu_f(r.z[kc][j]) : 1.f;
        }
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            *reinterpret_cast<float4*>(&s_dt[oc][ot + 4 * q]) =
                make_float4(vdt[4 * q], vdt[4 * q + 1], vdt[4 * q + 2], vdt[4 * q + 3]);
            *reinterpret_cast<float4*>(&s_dx[oc][ot + 4 * q]) =
                make_float4(vdx[4 * q], vdx[4 * q + 1], vdx[4 * q + 2], vdx[4 * q + 3]);
        }
        if (kc == 0) {
#pragma unroll
            for (int k = 0; k < BCE; ++k) {
                if (bc_slot[k] >= 0) {
                    const bool ok = bc_ok[k] && (F || tb + bc_t[k] < L);
                    (&s_B[0][0])[bc_slot[k]] = ok ? r.B[k] * kLn2 : 0.f;
                    (&s_C[0][0])[bc_slot[k]] = ok ? r.C[k] : 0.f;
                }
            }
        }
    };

    // TT recurrence steps of sub-tile kc; padded steps past the end have
    // dt = dt*u = 0 and leave h unchanged, so the loop never needs a bound check
    auto scan_tile = [&](int kc) __attribute__((always_inline)) {
        // the B / C broadcasts of step st are read two steps before their use
        // (at 8 states per wavefront the registers for that would spill)
        constexpr int PRE = SPW <= 4 ? 2 : 0;
        float bq[TT][SPW], cq[TT][SPW];
        auto read_bc = [&](int st) __attribute__((always_inline)) {
#pragma unroll
            for (int k = 0; k < SPW; ++k) {
                bq[st][k] = s_B[kc * TT + st][wave * SPW + k];
                cq[st][k] = s_C[kc * TT + st][wave * SPW + k];
            }
        };
#pragma unroll
        for (int st = 0; st < PRE; ++st) read_bc(st);
#pragma unroll
        for (int tt = 0; tt < TT; tt += 4) {
            const float4 dt4 = *reinterpret_cast<const float4*>(&s_dt[lane][tt]);
            const float4 dx4 = *reinterpret_cast<const float4*>(&s_dx[lane][tt]);
            const float dts[4] = {dt4.x, dt4.y, dt4.z, dt4.w};
            const float dxs[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
            float yq[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int st = tt + q;
                if (PRE > 0 && st + PRE < TT) read_bc(st + PRE);
                float acc = 0.f;
#pragma unroll
                for (int k = 0; k < SPW; ++k) {
                    const float bk = PRE > 0 ? bq[st][k] : s_B[kc * TT + st][wave * SPW + k];
                    const float ck = PRE > 0 ? cq[st][k] : s_C[kc * TT + st][wave * SPW + k];
                    h[k] = fmaf(__builtin_amdgcn_exp2f(dts[q] * a2[k]), h[k], dxs[q] * bk);
                    acc = fmaf(h[k], ck, acc);
                }
                yq[q] = acc;
            }
            *reinterpret_cast<float4*>(&s_y[wave][lane][tt]) = make_float4(yq[0], yq[1], yq[2], yq[3]);
        }
    };

    // y of sub-tile kc into registers; the whole load tile is stored after
    // its last sub-tile
    auto finish_tile = [&](int tb, int kc, auto full) __attribute__((always_inline)) {
        constexpr bool F = decltype(full)::value;
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            float4 acc = *reinterpret_cast<const float4*>(&s_y[0][oc][ot + 4 * q]);
#pragma unroll
            for (int w = 1; w < NW; ++w) {
                const float4 p = *reinterpret_cast<const float4*>(&s_y[w][oc][ot + 4 * q]);
                acc.x += p.x; acc.y += p.y; acc.z += p.z; acc.w += p.w;
            }
            yout[kc][4 * q] = fmaf(D_c, du[4 * q], acc.x) * gz[4 * q];
            yout[kc][4 * q + 1] = fmaf(D_c, du[4 * q + 1], acc.y) * gz[4 * q + 1];
            yout[kc][4 * q + 2] = fmaf(D_c, du[4 * q + 2], acc.z) * gz[4 * q + 2];
            yout[kc][4 * q + 3] = fmaf(D_c, du[4 * q + 3], acc.w) * gz[4 * q + 3];
        }
        if (kc != KC - 1 || !c_ok) return;
#pragma unroll
        for (int k2 = 0; k2 < KC; ++k2) {
            const int t0 = tb + k2 * TT + ot;
            if constexpr (CM && VEC) {
                const uint32_t so = (uint32_t)(tb + k2 * TT) * (uint32_t)sizeof(T);
                if constexpr (F) {
#pragma unroll
                    for (int q = 0; q < E / 4; ++q) Buf4<T>::store(ry_cm, vo_y + q * 4 * sizeof(T), so, &yout[k2][4 * q]);
                } else {
#pragma unroll
                    for (int j = 0; j < E; ++j)
                        if (t0 + j < L) BufAct<T>::store(ry_cm, vo_y + j * sizeof(T), so, yout[k2][j]);
                }
            } else if constexpr (CM && F) {
                store_run<T, E, VEC>(yp + t0, yout[k2]);
            } else if constexpr (CM) {
#pragma unroll
                for (int j = 0; j < E; ++j)
                    if (F || t0 + j < L) Act<T>::store(yp + t0 + j, yout[k2][j]);
            } else {
                const int tw = tb + k2 * TT + ot_u;
                if (F || tw < L) {
                    const auto ry = row_rsrc(yb + (int64_t)tw * a.y_sl, run_bytes_y);
#pragma unroll
                    for (int j = 0; j < E; ++j)
                        if (F || tw + j < L) BufAct<T>::store(ry, ch_bytes, (uint32_t)j * sl_bytes_y, yout[k2][j]);
                }
            }
        }
    };

    // refill(kc) runs once sub-tile kc is staged, when its raw registers are free
    auto run_subtiles = [&](Raw& r, int tb, auto full, auto refill) __attribute__((always_inline)) {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            stage_tile(r, tb, kc, full);
            __syncthreads();
            refill(kc);
            scan_tile(kc);
            __syncthreads();
            finish_tile(tb, kc, full);
        }
    };

    // Only full load tiles pass through the pipeline, so the loads have a
    // single code path (two paths would merge through register copies that
    // wait for the loads).  The refill is unconditional: the last tiles
    // re-read tile nfull-1 rather than branch.  Token-major keeps two raw
    // sets (the tile two ahead in flight).  Channel-major load tiles are
    // twice as long and hold one set within the 3-waves-per-SIMD register
    // budget: each sub-tile's registers are refilled with the same sub-tile
    // of the next load tile as soon as it is staged (B/C with sub-tile 0), so
    // every load is in flight across two sub-tile scans (refilling the whole
    // tile after its last sub-tile gave the first half one scan: 3% slower).
    const int nfull = L / LT;
    // Issue priority falls as the sequence progresses (levels change at 1/2,
    // 3/4 and 7/8 of the load tiles).  The SIMDs issue oldest-wave-first, so
    // without this the first workgroup resident on a CU runs far ahead and
    // the last one finishes alone at low occupancy; with it, a workgroup
    // that got ahead yields its issue slots to the ones behind it on the same
    // CU at each level change, and the final level (where the spread builds
    // up again) is only an eighth of the sequence.
    auto set_prio = [&](int i) __attribute__((always_inline)) {
        const int n8 = 8 * i, nf = max(nfull, 1);
        const int lvl = n8 < 4 * nf ? 0 : n8 < 6 * nf ? 1 : n8 < 7 * nf ? 2 : 3;
        if (lvl == 0) __builtin_amdgcn_s_setprio(3);
        else if (lvl == 1) __builtin_amdgcn_s_setprio(2);
        else if (lvl == 2) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
    };
    if constexpr (KC == 1) {
        auto run_full = [&](Raw& r, int i) __attribute__((always_inline)) {
            set_prio(i);
            run_subtiles(r, i * LT, Full<true>{},
                         [&](int) { load_tile(r, min(i + 2, nfull - 1) * LT, Full<true>{}); });
        };
        if (nfull > 0) load_tile(r0, 0, Full<true>{});
        if (nfull > 1) load_tile(r1, LT, Full<true>{});
        int i = 0;
        for (; i + 1 < nfull; i += 2) {
            run_full(r0, i);
            run_full(r1, i + 1);
        }
        if (i < nfull) run_full(r0, i);
    } else {
        // two load tiles per iteration: the loop-carried registers then line
        // up at the back edge without copies
        auto run_cm = [&](int i) __attribute__((always_inline)) {
            set_prio(i);
            const int nb = min(i + 1, nfull - 1) * LT;
            run_subtiles(r0, i * LT, Full<true>{}, [&](int kc) {
                load_sub(r0, nb, kc, Full<true>{});
                if (kc == 0) load_bc(r0, nb, Full<true>{});
            });
        };
        if (nfull > 0) load_tile(r0, 0, Full<true>{});
        int i = 0;
        for (; i + 1 < nfull; i += 2) {
            run_cm(i);
            run_cm(i + 1);
        }
        if (i < nfull) run_cm(i);
    }
    if (nfull * LT < L) {  // the partial last load tile, outside the pipeline
        const int tb = nfull * LT;
        load_tile(r0, tb, Full<false>{});
        run_subtiles(r0, tb, Full<false>{}, [](int) {});
    }

    if (a.h_out) {
#pragma unroll
        for (int k = 0; k < SPW; ++k) {
            const int n = wave * SPW + k;
            if (lane_ok && n < N) a.h_out[((int64_t)b * D + c0 + lane) * N + n] = h[k];
        }
    }
}

template <typename T, int NW, int SPW, int TT, bool CM, bool VEC>
void launch_scan(const ScanArgs& a, int64_t batch, hipStream_t st) {
    dim3 grid((unsigned)((a.D + 63) / 64), (unsigned)batch);
    if (a.softplus && a.z != nullptr)
        hipLaunchKernelGGL((scan_fwd_kernel<T, NW, SPW, TT, CM, VEC, false>), grid, dim3(NW * 64), 0, st, a);
    else
        hipLaunchKernelGGL((scan_fwd_kernel<T, NW, SPW, TT, CM, VEC, true>), grid, dim3(NW * 64), 0, st, a);
}

// ---------------------------------------------------------------------------
// Chunked scan across the lanes of a wavefront, for grids that leave the GPU
// mostly idle (few batch rows x 64-channel blocks): the tiled kernel above
// walks every step of a sequence in turn, so its time is the sequence length
// times the latency of one step whatever the size of the grid.  Here one
// wavefront owns one (batch row, channel), and its 64 lanes hold 64
// consecutive steps -- a chunk.  For each state n the recurrence
//   h_t = dA_t h_{t-1} + dBx_t
// is the composition of the affine maps (dA_t, dBx_t), and
//   (a1, b1) then (a2, b2) = (a2 a1, a2 b1 + b2)
// is associative, so an inclusive scan over the lanes gives every step's
// (prod of dA, h from a zero start) at once: six DPP levels (row_shr 1, 2, 4,
// 8 within each 16-lane row, then row_bcast 15 and 31 across rows), each
// lane combining with the identity (1, 0) where it has no source.  The state
// entering the chunk is then folded in as h_t = P_t h_in + h_t, and lane 63's
// h (identical to the last valid step's: steps past the end are identity
// maps with dt = 0) is carried into the next chunk -- the (prod dA, h) carry
// of a chunked scan.  The order of every operation is fixed, so results are
// deterministic; the tree order of the scan rounds differently from the
// step-by-step loop (within fp32 rounding of it).
// The eight wavefronts of a workgroup take eight consecutive channels of one
// batch row, share each chunk's B and C tiles through LDS, and move their u,
// delta, z and y tiles through LDS as well (coalesced in either layout).
constexpr int kLaneChannels = 8;   // wavefronts (channels) per workgroup

// One level of the inclusive scan, for the four states of a group at once:
// (a, b) <- (source lane's map) then (a, b), i.e. b += b_src * a, a *= a_src.
// Each is one VOP2 instruction with a DPP source (v_fmac_f32_dpp,
// v_mul_f32_dpp) written in place: a lane with no source in this level (the
// first lanes of a row for row_shr; the rows row_mask leaves out for
// row_bcast) is not written, which is the identity map (1, 0) without a
// register to hold it.  b is updated before a, as it needs a's old value.
// The compiler's hazard checks do not see into asm, so the DPP read-after-
// VALU-write distance (2 wait states on gfx9) is kept by the interleave: the
// four chains put 7 instructions between a write and the next level's DPP
// read of the same register, and an s_nop guards the first level.
#define MTL_SCAN_LEVEL4(DPP)                                                                               \
    asm volatile("v_fmac_f32_dpp %0, %0, %4 " DPP "\n\t"                                                  \
                 "v_mul_f32_dpp %4, %4, %4 " DPP "\n\t"                                                   \
                 "v_fmac_f32_dpp %1, %1, %5 " DPP "\n\t"                                                  \
                 "v_mul_f32_dpp %5, %5, %5 " DPP "\n\t"                                                   \
                 "v_fmac_f32_dpp %2, %2, %6 " DPP "\n\t"                                                  \
                 "v_mul_f32_dpp %6, %6, %6 " DPP "\n\t"                                                   \
                 "v_fmac_f32_dpp %3, %3, %7 " DPP "\n\t"                                                  \
                 "v_mul_f32_dpp %7, %7, %7 " DPP                                                            \
                 : "+v"(bv[0]), "+v"(bv[1]), "+v"(bv[2]), "+v"(bv[3]), "+v"(av[0]), "+v"(av[1]), "+v"(av[2]), \
                   "+v"(av[3]))

template <typename T, int NS>
__global__ void __launch_bounds__(kLaneChannels * 64) scan_lanes_kernel(const ScanArgs a) {
    constexpr int CW = kLaneChannels, NT = CW * 64;
    __shared__ float s_B[NS][65];                      // padded rows: the state-fastest fill hits distinct banks
    __shared__ float s_C[NS][65];
    __shared__ float s_x[3][CW][65];                   // u, delta, z of the workgroup's channels, then y
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b = blockIdx.y;
    const int L = a.L, D = a.D, N = a.N;
    const int c0 = blockIdx.x * CW;
    const int c_raw = c0 + wave;
    const bool c_ok = c_raw < D;                       // waves past D still take part in the barriers
    const int c = c_ok ? c_raw : D - 1;
    const bool has_z = a.z != nullptr;

    // The workgroup's u, delta, z (and y) tiles of CW channels x 64 steps move
    // between HBM and LDS cooperatively: with unit step stride thread e takes
    // channel e / 64, step e % 64; otherwise (token-major rows) step e / CW,
    // channel e % CW, so a wavefront reads whole CW-channel runs of 64 / CW rows
    // instead of one word of 64 rows.  Wavefront w then works on channel w
    // with lane = step.
    const bool x_t_fast = a.u_sl == 1;
    const int xe_c = x_t_fast ? tid >> 6 : tid % CW, xe_t = x_t_fast ? tid & 63 : tid / CW;
    const int xc = min(c0 + xe_c, D - 1);
    const T* up = static_cast<const T*>(a.u) + b * a.u_sb + (int64_t)xc * a.u_sd;
    const T* dp = static_cast<const T*>(a.delta) + b * a.d_sb + (int64_t)xc * a.d_sd;
    const T* zp = has_z ? static_cast<const T*>(a.z) + b * a.z_sb + (int64_t)xc * a.z_sd : up;
    const int64_t z_sl = has_z ? a.z_sl : a.u_sl;
    T* yp = static_cast<T*>(a.y) + b * a.y_sb + (int64_t)xc * a.y_sd;
    const bool xc_ok = c0 + xe_c < D;
    const T* Bp = static_cast<const T*>(a.B) + b * a.B_sb;
    const T* Cp = static_cast<const T*>(a.C) + b * a.C_sb;

    constexpr int kFill = (NS * 64 + NT - 1) / NT;     // B and C values each thread stages per chunk
    // B/C tile element e of a chunk: state n, step tl.  With unit step stride
    // consecutive threads take consecutive steps; otherwise (B and C as
    // columns of the token-major x_dbl) consecutive states.
    const bool bc_t_fast = a.B_sl == 1;
    struct Chunk { float fb[kFill], fc[kFill], u, d, z; };
    auto load_chunk = [&](Chunk& k, int t0) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < kFill; ++q) {
            const int e = min(tid + q * NT, NS * 64 - 1);
            const int n = bc_t_fast ? e >> 6 : e % NS, tl = bc_t_fast ? e & 63 : e / NS;
            const int tcq = min(t0 + tl, L - 1), nn = min(n, N - 1);
            k.fb[q] = Act<T>::load(Bp + (int64_t)nn * a.B_sn + (int64_t)tcq * a.B_sl);
            k.fc[q] = Act<T>::load(Cp + (int64_t)nn * a.C_sn + (int64_t)tcq * a.C_sl);
        }
        const int tc = min(t0 + xe_t, L - 1);
        k.u = Act<T>::load(up + (int64_t)tc * a.u_sl);
        k.d = Act<T>::load(dp + (int64_t)tc * a.d_sl);
        k.z = Act<T>::load(zp + (int64_t)tc * z_sl);
    };
    // software pipeline: the next chunk's loads are in flight while this one is scanned
    Chunk cur, nxt;
    load_chunk(cur, 0);

    // (after the first chunk's loads are issued, so the two round trips overlap)
    // lane n < N fetches state n's A (and h0) once; every lane then reads
    // them out uniformly.  States n >= N have A = 0 and B = C = 0: identity
    // maps that add nothing, so the state loop needs no branch and its
    // chains interleave.
    const float bias_l2 = (a.dbias ? a.dbias[c] : 0.f) * kLog2e;
    const float D_c = a.Dv ? a.Dv[c] : 0.f;
    const int nl = min(lane, N - 1);
    float a_lane = a.A[(int64_t)c * N + nl];
    if (a.a_is_log) a_lane = -expf(a_lane);
    a_lane = lane < N ? a_lane : 0.f;
    float h_lane = a.h0 ? a.h0[((int64_t)b * D + c) * N + nl] : 0.f;
    h_lane = lane < N ? h_lane : 0.f;
    float A_c[NS], h_in[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n) {
        A_c[n] = lane_read(a_lane, n);
        h_in[n] = lane_read(h_lane, n);
    }

    for (int t0 = 0; t0 < L; t0 += 64) {
#pragma unroll
        for (int q = 0; q < kFill; ++q) {
            const int e = tid + q * NT;
            if (NS * 64 % NT == 0 || e < NS * 64) {
                const int n = bc_t_fast ? e >> 6 : e % NS, tl = bc_t_fast ? e & 63 : e / NS;
                s_B[n][tl] = n < N ? cur.fb[q] : 0.f;  // padded states: identity, no output
                s_C[n][tl] = n < N ? cur.fc[q] : 0.f;
            }
        }
        s_x[0][xe_c][xe_t] = cur.u;
        s_x[1][xe_c][xe_t] = cur.d;
        s_x[2][xe_c][xe_t] = cur.z;
        // the next chunk's loads only when there is one: a last chunk that
        // re-read itself made every wavefront wait for those loads before
        // exiting (64-token prompt: 4.94 -> 4.76 us per launch)
        if (t0 + 64 < L) load_chunk(nxt, t0 + 64);
        __syncthreads();
        const int t = t0 + lane;
        const bool valid = t < L;
        const float uv = s_x[0][wave][lane], zv = s_x[2][wave][lane];
        float dt = fmaf(s_x[1][wave][lane], kLog2e, bias_l2);   // log2 units
        if (a.softplus) dt = softplus_l2_f(dt);
        dt = valid ? dt : 0.f;                         // identity map past the end
        const float dx = dt * kLn2 * uv;               // dt (natural units) * u
        float yacc = 0.f;
        // states in groups of four: each level of the four scans is issued
        // together, so one chain's DPP latency is covered by the others
#pragma unroll
        for (int n0 = 0; n0 < NS; n0 += 4) {
            float av[4], bv[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                av[k] = __builtin_amdgcn_exp2f(dt * A_c[n0 + k]);
                bv[k] = dx * s_B[n0 + k][lane];
            }
            asm volatile("s_nop 2" ::: "memory");
            MTL_SCAN_LEVEL4("row_shr:1 row_mask:0xf bank_mask:0xf");
            MTL_SCAN_LEVEL4("row_shr:2 row_mask:0xf bank_mask:0xf");
            MTL_SCAN_LEVEL4("row_shr:4 row_mask:0xf bank_mask:0xf");
            MTL_SCAN_LEVEL4("row_shr:8 row_mask:0xf bank_mask:0xf");
            MTL_SCAN_LEVEL4("row_bcast:15 row_mask:0xa bank_mask:0xf");
            MTL_SCAN_LEVEL4("row_bcast:31 row_mask:0xc bank_mask:0xf");
            asm volatile("s_nop 1" ::: "memory");
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float hv = fmaf(av[k], h_in[n0 + k], bv[k]);
                yacc = fmaf(s_C[n0 + k][lane], hv, yacc);
                h_in[n0 + k] = lane_read(hv, 63);
            }
        }
        const float yv = fmaf(D_c, uv, yacc) * (has_z ? silu_f(zv) : 1.f);
        __syncthreads();                               // every wavefront has read its u, delta, z
        s_x[0][wave][lane] = yv;
        __syncthreads();
        const int ty = t0 + xe_t;
        if (xc_ok && ty < L) Act<T>::store(yp + (int64_t)ty * a.y_sl, s_x[0][xe_c][xe_t]);
        cur = nxt;
    }
    if (a.h_out && c_ok) {
        float hv = 0.f;
#pragma unroll
        for (int n = 0; n < NS; ++n) hv = lane == n ? h_in[n] : hv;
        if (lane < N) a.h_out[((int64_t)b * D + c) * N + lane] = hv;
    }
}

// Long sequences on the same grids: each lane holds kLaneSteps consecutive
// steps, so a chunk is 64 kLaneSteps steps.  Per state, a lane first folds
// its steps into one affine map (pass 1: the product of their dA and the h
// they make from a zero start), the six DPP levels scan those maps across
// the lanes as above, lane l takes lane l - 1's end state (wave_shr:1; lane
// 0 the chunk's incoming state) and walks its steps again from it (pass 2),
// accumulating C . h per step.  The scan's 12 DPP instructions per state are
// then spent once per kLaneSteps steps, and a chunk's barriers and staging
// once per 256 steps.  Fixed order throughout: deterministic, within fp32
// rounding of the step-by-step loop.
// It holds more registers (NS = 16: 214 VGPRs, one 8-wavefront workgroup per
// CU), so it is taken where the grid is one workgroup per CU at most, for
// sequences over 128 steps and 5 to 16 states.  Measured against the
// kernel above (mixer layout, HIP events): D 1536, batch 1, 1024 steps 35.5
// -> 28.6 us, 256 steps 11.0 -> 8.4 us; bf16 D 2048, 2048 steps 81.1 -> 59.9
// us; at 512 workgroups (D 4096) 60.7 -> 58.8 us but 104.6 -> 111.2 us at
// batch 2, D 2048; with 4 states 13.0 -> 14.5 us.
constexpr int kLaneSteps = 4;
constexpr int kLanesLongMinSteps = 128;
constexpr int64_t kLanesLongMaxWorkgroups = 256;
constexpr int kLanesLongMinStates = 5;
constexpr int kLanesLongMaxStates = 16;     // 32 states would spill (256 VGPRs and scratch)

template <typename T, int NS>
__global__ void __launch_bounds__(kLaneChannels * 64) scan_lanes_long_kernel(const ScanArgs a) {
    constexpr int CW = kLaneChannels, NT = CW * 64, S = kLaneSteps, CH = 64 * S;
    constexpr int RS = CH + 4;                          // LDS row stride: 16-byte aligned, a state-fastest fill spreads over banks
    static_assert(S == 4, "a lane's steps are one float4 of an LDS row");
    __shared__ __align__(16) float s_B[NS][RS];
    __shared__ __align__(16) float s_C[NS][RS];
    __shared__ __align__(16) float s_x[3][CW][RS];       // u, delta, z of the workgroup's channels, then y
    // each wavefront's A and carried state per state: the state-group loop
    // stays rolled (one group's S x 4 maps live at a time), so they are read
    // from LDS per group rather than held in registers
    __shared__ __align__(16) float s_A[CW][NS];
    __shared__ __align__(16) float s_h[CW][NS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b = blockIdx.y;
    const int L = a.L, D = a.D, N = a.N;
    const int c0 = blockIdx.x * CW;
    const int c_raw = c0 + wave;
    const bool c_ok = c_raw < D;                       // waves past D still take part in the barriers
    const int c = c_ok ? c_raw : D - 1;
    const bool has_z = a.z != nullptr;

    // u, delta, z (and y) tiles of CW channels x CH steps, moved cooperatively:
    // element e of the tile is (channel, step) = (e / CH, e % CH) with unit step
    // stride, else (e % CW, e / CW), so consecutive threads touch consecutive
    // addresses either way
    constexpr int XE = CW * CH / NT;                   // tile elements per thread
    const bool x_t_fast = a.u_sl == 1;
    const T* ub = static_cast<const T*>(a.u) + b * a.u_sb;
    const T* db = static_cast<const T*>(a.delta) + b * a.d_sb;
    const T* zb = has_z ? static_cast<const T*>(a.z) + b * a.z_sb : ub;
    const int64_t z_sd = has_z ? a.z_sd : a.u_sd, z_sl = has_z ? a.z_sl : a.u_sl;
    T* yb = static_cast<T*>(a.y) + b * a.y_sb;
    const T* Bp = static_cast<const T*>(a.B) + b * a.B_sb;
    const T* Cp = static_cast<const T*>(a.C) + b * a.C_sb;
    auto xe_ct = [&](int q, int& ce, int& te) __attribute__((always_inline)) {
        const int e = tid + q * NT;
        ce = x_t_fast ? e / CH : e % CW;
        te = x_t_fast ? e % CH : e / CW;
    };

    constexpr int kFill = (NS * CH + NT - 1) / NT;     // B and C values each thread stages per chunk
    const bool bc_t_fast = a.B_sl == 1;
    struct Chunk { float fb[kFill], fc[kFill], u[XE], d[XE], z[XE]; };
    auto load_chunk = [&](Chunk& k, int t0) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < kFill; ++q) {
            const int e = min(tid + q * NT, NS * CH - 1);
            const int n = bc_t_fast ? e / CH : e % NS, tl = bc_t_fast ? e % CH : e / NS;
            const int tcq = min(t0 + tl, L - 1), nn = min(n, N - 1);
            k.fb[q] = Act<T>::load(Bp + (int64_t)nn * a.B_sn + (int64_t)tcq * a.B_sl);
            k.fc[q] = Act<T>::load(Cp + (int64_t)nn * a.C_sn + (int64_t)tcq * a.C_sl);
        }
#pragma unroll
        for (int q = 0; q < XE; ++q) {
            int ce, te;
            xe_ct(q, ce, te);
            const int64_t cc = min(c0 + ce, D - 1), tc = min(t0 + te, L - 1);
            k.u[q] = Act<T>::load(ub + cc * a.u_sd + tc * a.u_sl);
            k.d[q] = Act<T>::load(db + cc * a.d_sd + tc * a.d_sl);
            k.z[q] = Act<T>::load(zb + cc * z_sd + tc * z_sl);
        }
    };
    Chunk cur, nxt;
    load_chunk(cur, 0);

    const float bias_l2 = (a.dbias ? a.dbias[c] : 0.f) * kLog2e;
    const float D_c = a.Dv ? a.Dv[c] : 0.f;
    const int nl = min(lane, N - 1);
    float a_lane = a.A[(int64_t)c * N + nl];
    if (a.a_is_log) a_lane = -expf(a_lane);
    a_lane = lane < N ? a_lane : 0.f;
    float h_lane = a.h0 ? a.h0[((int64_t)b * D + c) * N + nl] : 0.f;
    h_lane = lane < N ? h_lane : 0.f;
    if (lane < NS) {
        s_A[wave][lane] = a_lane;
        s_h[wave][lane] = h_lane;
    }

    for (int t0 = 0; t0 < L; t0 += CH) {
#pragma unroll
        for (int q = 0; q < kFill; ++q) {
            const int e = tid + q * NT;
            if (NS * CH % NT == 0 || e < NS * CH) {
                const int n = bc_t_fast ? e / CH : e % NS, tl = bc_t_fast ? e % CH : e / NS;
                s_B[n][tl] = n < N ? cur.fb[q] : 0.f;  // padded states: identity, no output
                s_C[n][tl] = n < N ? cur.fc[q] : 0.f;
            }
        }
#pragma unroll
        for (int q = 0; q < XE; ++q) {
            int ce, te;
            xe_ct(q, ce, te);
            s_x[0][ce][te] = cur.u[q];
            s_x[1][ce][te] = cur.d[q];
            s_x[2][ce][te] = cur.z[q];
        }
        if (t0 + CH < L) load_chunk(nxt, t0 + CH);
        __syncthreads();
        // this lane's steps t0 + S lane + s
        const float4 u4 = *reinterpret_cast<const float4*>(&s_x[0][wave][S * lane]);
        const float4 d4 = *reinterpret_cast<const float4*>(&s_x[1][wave][S * lane]);
        const float4 z4 = *reinterpret_cast<const float4*>(&s_x[2][wave][S * lane]);
        const float uv[S] = {u4.x, u4.y, u4.z, u4.w}, dv[S] = {d4.x, d4.y, d4.z, d4.w},
                    zv[S] = {z4.x, z4.y, z4.z, z4.w};
        float dt[S], dx[S], yacc[S];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            float v = fmaf(dv[s], kLog2e, bias_l2);     // log2 units
            if (a.softplus) v = softplus_l2_f(v);
            v = t0 + S * lane + s < L ? v : 0.f;        // identity map past the end
            dt[s] = v;
            dx[s] = v * kLn2 * uv[s];                   // dt (natural units) * u
            yacc[s] = 0.f;
        }
#pragma unroll 1
        for (int n0 = 0; n0 < NS; n0 += 4) {
            const float4 A4 = *reinterpret_cast<const float4*>(&s_A[wave][n0]);
            const float4 H4 = *reinterpret_cast<const float4*>(&s_h[wave][n0]);
            const float Ag[4] = {A4.x, A4.y, A4.z, A4.w}, Hg[4] = {H4.x, H4.y, H4.z, H4.w};
            // pass 1: each state's S steps folded into one map (av, bv)
            float dA[4][S], dB[4][S], av[4], bv[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 B4 = *reinterpret_cast<const float4*>(&s_B[n0 + k][S * lane]);
                const float Bs[S] = {B4.x, B4.y, B4.z, B4.w};
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    dA[k][s] = __builtin_amdgcn_exp2f(dt[s] * Ag[k]);
                    dB[k][s] = dx[s] * Bs[s];
                }
                float pa = dA[k][0], pb = dB[k][0];
#pragma unroll
                for (int s = 1; s < S; ++s) {
                    pb = fmaf(dA[k][s], pb, dB[k][s]);
                    pa = pa * dA[k][s];
                }
                av[k] = pa;
                bv[k] = pb;
            }
            asm volatile("s_nop 2" ::: "memory");
            MTL_SCAN_LEVEL4("row_shr:1 row_mask:0xf bank_mask:0xf");
            MTL_SCAN_LEVEL4("row_shr:2 row_mask:0xf bank_mask:0xf");
            MTL_SCAN_LEVEL4("row_shr:4 row_mask:0xf bank_mask:0xf");
            MTL_SCAN_LEVEL4("row_shr:8 row_mask:0xf bank_mask:0xf");
            MTL_SCAN_LEVEL4("row_bcast:15 row_mask:0xa bank_mask:0xf");
            MTL_SCAN_LEVEL4("row_bcast:31 row_mask:0xc bank_mask:0xf");
            asm volatile("s_nop 1" ::: "memory");
            // pass 2: from the end state of lane l - 1 (the chunk's incoming
            // state for lane 0) through this lane's steps
            float hnext[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float h_end = fmaf(av[k], Hg[k], bv[k]);
                float h = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                    __builtin_bit_cast(int, Hg[k]), __builtin_bit_cast(int, h_end), kDppWaveShr1, 0xf, 0xf,
                    false));
                const float4 C4 = *reinterpret_cast<const float4*>(&s_C[n0 + k][S * lane]);
                const float Cs[S] = {C4.x, C4.y, C4.z, C4.w};
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    h = fmaf(dA[k][s], h, dB[k][s]);
                    yacc[s] = fmaf(Cs[s], h, yacc[s]);
                }
                hnext[k] = lane_read(h_end, 63);
            }
            // every lane has read the group's old states above (LDS operations
            // of one wavefront complete in order)
            if (lane == 0)
                *reinterpret_cast<float4*>(&s_h[wave][n0]) = make_float4(hnext[0], hnext[1], hnext[2], hnext[3]);
        }
        float yv[S];
#pragma unroll
        for (int s = 0; s < S; ++s) yv[s] = fmaf(D_c, uv[s], yacc[s]) * (has_z ? silu_f(zv[s]) : 1.f);
        __syncthreads();                               // every wavefront has read its u, delta, z
        *reinterpret_cast<float4*>(&s_x[0][wave][S * lane]) = make_float4(yv[0], yv[1], yv[2], yv[3]);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < XE; ++q) {
            int ce, te;
            xe_ct(q, ce, te);
            if (c0 + ce < D && t0 + te < L)
                Act<T>::store(yb + (int64_t)(c0 + ce) * a.y_sd + (int64_t)(t0 + te) * a.y_sl, s_x[0][ce][te]);
        }
        cur = nxt;
    }
    if (a.h_out && c_ok && lane < N) a.h_out[((int64_t)b * D + c) * N + lane] = s_h[wave][lane];
}

template <typename T>
void launch_scan_lanes(const ScanArgs& a, int64_t batch, hipStream_t st) {
    dim3 grid((unsigned)((a.D + kLaneChannels - 1) / kLaneChannels), (unsigned)batch);
    dim3 block(kLaneChannels * 64);
    if (a.L > kLanesLongMinSteps && a.N >= kLanesLongMinStates && a.N <= kLanesLongMaxStates &&
        (int64_t)grid.x * grid.y <= kLanesLongMaxWorkgroups) {
        if (a.N <= 8) hipLaunchKernelGGL((scan_lanes_long_kernel<T, 8>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((scan_lanes_long_kernel<T, 16>), grid, block, 0, st, a);
        return;
    }
    if (a.N <= 4) hipLaunchKernelGGL((scan_lanes_kernel<T, 4>), grid, block, 0, st, a);
    else if (a.N <= 8) hipLaunchKernelGGL((scan_lanes_kernel<T, 8>), grid, block, 0, st, a);
    else if (a.N <= 16) hipLaunchKernelGGL((scan_lanes_kernel<T, 16>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((scan_lanes_kernel<T, 32>), grid, block, 0, st, a);
}

// algo 0 takes the chunked kernel when the tiled kernel's grid (batch *
// ceil(D / 64) workgroups of 4 wavefronts) is below this and the sequence is
// longer than kChunkedMinSteps.  Measured on MI355X as HIP-graph replays,
// mixer layout, fp32: the chunked kernel wins from 12 to 128 workgroups at
// 64 steps and more (D 1536, 64 steps, batch 1: 5.4 against 11.2 us; 1024
// steps: 37 against 126 us; D 4096, batch 2, 64 steps: a tie) and loses from
// 192 workgroups on, and at 16 steps, where both are at launch latency.
constexpr int64_t kChunkedBelowWorkgroups = 160;
constexpr int64_t kChunkedMinSteps = 32;

// 4 state groups of ceil(N/4) states: 4 wavefronts of 64 channels
template <typename T, bool CM, bool VEC>
void dispatch_spw(const ScanArgs& a, int64_t batch, hipStream_t st) {
    if (a.N <= 4) launch_scan<T, 4, 1, 16, CM, VEC>(a, batch, st);
    else if (a.N <= 8) launch_scan<T, 4, 2, 16, CM, VEC>(a, batch, st);
    else if (a.N <= 16) launch_scan<T, 4, 4, 16, CM, VEC>(a, batch, st);
    else launch_scan<T, 4, 8, 16, CM, VEC>(a, batch, st);
}

template <typename T>
bool rows_aligned(const ScanArgs& a, int64_t batch) {
    const uintptr_t al = sizeof(T) == 4 ? 16 : 8;
    auto ok = [&](const void* p, int64_t sb, int64_t sd) {
        return p == nullptr || ((uintptr_t)p % al == 0 && (batch == 1 || (sb * (int64_t)sizeof(T)) % al == 0) &&
                                (sd * (int64_t)sizeof(T)) % al == 0);
    };
    auto span = [&](const void* p, int64_t sd) {
        return p == nullptr || ((int64_t)(a.D - 1) * sd + a.L) * (int64_t)sizeof(T) < (int64_t(1) << 31);
    };
    return ok(a.u, a.u_sb, a.u_sd) && ok(a.delta, a.d_sb, a.d_sd) && ok(a.z, a.z_sb, a.z_sd) &&
           ok(a.y, a.y_sb, a.y_sd) && span(a.u, a.u_sd) && span(a.delta, a.d_sd) && span(a.z, a.z_sd) &&
           span(a.y, a.y_sd);
}

}  // namespace
}  // namespace mtl

extern "C" int mtl_selective_scan_fwd(const mtl_scan_params* p, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(p != nullptr, "null params");
    MTL_REQUIRE(p->batch >= 0 && p->seqlen >= 0 && p->dim >= 0, "negative size");
    MTL_REQUIRE(p->dstate >= 1 && p->dstate <= 32, "dstate must be in [1, 32]");
    MTL_REQUIRE(p->batch <= 65535, "batch must be <= 65535");
    MTL_REQUIRE(p->batch * ((p->dim + 63) / 64) < (int64_t(1) << 31), "batch * ceil(dim / 64) overflows int32");
    MTL_REQUIRE(p->seqlen < (int64_t(1) << 31) && p->dim < (int64_t(1) << 31), "size overflows int32");
    MTL_REQUIRE(p->dtype == MTL_F32 || p->dtype == MTL_BF16, "dtype must be MTL_F32 or MTL_BF16");
    if (p->batch == 0 || p->dim == 0) return MTL_OK;
    MTL_REQUIRE(p->A != nullptr, "null A");
    // an empty sequence only carries h0 (or zeros) through to h_out; torch
    // hands out null data pointers for empty tensors
    MTL_REQUIRE(p->seqlen == 0 || (p->u && p->delta && p->B && p->C && p->y), "null required pointer");

    const bool has_z = p->z != nullptr;
    const bool cm = p->u_sl == 1 && p->delta_sl == 1 && p->y_sl == 1 && (!has_z || p->z_sl == 1);
    const bool tm = p->u_sd == 1 && p->delta_sd == 1 && p->y_sd == 1 && (!has_z || p->z_sd == 1);
    MTL_REQUIRE(cm || tm || p->seqlen <= 1,
                "u/delta/z/y must all be channel-major (stride_l == 1) or all token-major (stride_d == 1)");

    ScanArgs a;
    a.u = p->u; a.delta = p->delta; a.z = p->z; a.B = p->B; a.C = p->C; a.y = p->y;
    a.A = p->A; a.Dv = p->D; a.dbias = p->delta_bias; a.h0 = p->h0; a.h_out = p->h_out;
    a.u_sb = p->u_sb; a.u_sd = p->u_sd; a.u_sl = p->u_sl;
    a.d_sb = p->delta_sb; a.d_sd = p->delta_sd; a.d_sl = p->delta_sl;
    a.z_sb = p->z_sb; a.z_sd = p->z_sd; a.z_sl = p->z_sl;
    a.B_sb = p->B_sb; a.B_sn = p->B_sn; a.B_sl = p->B_sl;
    a.C_sb = p->C_sb; a.C_sn = p->C_sn; a.C_sl = p->C_sl;
    a.y_sb = p->y_sb; a.y_sd = p->y_sd; a.y_sl = p->y_sl;
    a.L = (int)p->seqlen; a.D = (int)p->dim; a.N = (int)p->dstate;
    a.softplus = p->delta_softplus; a.a_is_log = p->a_is_log;
    // B/C element offsets within a load tile and token-major channel offsets
    // are 32-bit byte offsets (non-negative strides, spans under 4 GiB)
    MTL_REQUIRE(p->B_sn >= 0 && p->B_sl >= 0 && p->C_sn >= 0 && p->C_sl >= 0, "negative B/C stride");
    {
        const int64_t es = p->dtype == MTL_F32 ? 4 : 2, lt = std::min<int64_t>(32, std::max<int64_t>(p->seqlen, 1));
        const int64_t span_b = ((p->dstate - 1) * p->B_sn + (lt - 1) * p->B_sl + 1) * es;
        const int64_t span_c = ((p->dstate - 1) * p->C_sn + (lt - 1) * p->C_sl + 1) * es;
        MTL_REQUIRE(span_b < (int64_t(1) << 32) && span_c < (int64_t(1) << 32), "B/C strides too large");
        MTL_REQUIRE(p->dim * es < (int64_t(1) << 32), "dim too large");
        // token-major runs are addressed through buffer resources spanning
        // (run - 1) row strides + one row (the run is at most 8 steps)
        if (!(p->u_sl == 1 && p->delta_sl == 1 && p->y_sl == 1) && p->seqlen > 1) {
            const int64_t sl_max = std::max({p->u_sl, p->delta_sl, p->y_sl, p->z ? p->z_sl : p->u_sl});
            MTL_REQUIRE(p->u_sl >= 0 && p->delta_sl >= 0 && p->y_sl >= 0 && (!p->z || p->z_sl >= 0),
                        "negative step stride");
            MTL_REQUIRE((7 * sl_max + p->dim) * es < (int64_t(1) << 31), "token-major step stride too large");
        }
    }

    MTL_REQUIRE(p->algo >= 0 && p->algo <= 2, "algo must be 0 (auto), 1 (tiled) or 2 (chunked)");
    hipStream_t st = as_stream(stream);
    if (p->seqlen == 0) {
        // no steps: h_out = h0 (or zeros); the tiled kernel's path carries it
    } else if (p->algo == 2 || (p->algo == 0 && p->batch * ((p->dim + 63) / 64) < kChunkedBelowWorkgroups &&
                                p->seqlen > kChunkedMinSteps)) {
        MTL_REQUIRE(p->batch * ((p->dim + kLaneChannels - 1) / kLaneChannels) < (int64_t(1) << 31), "grid too large");
        if (p->dtype == MTL_F32) launch_scan_lanes<float>(a, p->batch, st);
        else launch_scan_lanes<uint16_t>(a, p->batch, st);
        return check_launch("selective_scan_fwd(chunked)");
    }
    // seqlen <= 1 has no meaningful l-stride; the channel-major path handles it.
    const bool use_cm = cm || (!tm);
    if (p->dtype == MTL_F32) {
        if (!use_cm) dispatch_spw<float, false, false>(a, p->batch, st);
        else if (rows_aligned<float>(a, p->batch)) dispatch_spw<float, true, true>(a, p->batch, st);
        else dispatch_spw<float, true, false>(a, p->batch, st);
    } else {
        if (!use_cm) dispatch_spw<uint16_t, false, false>(a, p->batch, st);
        else if (rows_aligned<uint16_t>(a, p->batch)) dispatch_spw<uint16_t, true, true>(a, p->batch, st);
        else dispatch_spw<uint16_t, true, false>(a, p->batch, st);
    }
    return check_launch("selective_scan_fwd");
}
