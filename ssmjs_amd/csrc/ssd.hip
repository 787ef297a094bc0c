// K3-K6: Mamba-2 SSD prefill (Dao & Gu 2024, section 6) for gfx950, and K7: the one-token
// Mamba-2 state update.
//
// This file: bf16 inputs (x, B, C; dt and y fp32). fp32 inputs run the fp32 matrix-core
// kernel of ssd_f32.hip. One workgroup owns one (batch, segment) and HPW heads of one group (4
// waves per head; two heads when heads pair up in a group) and walks the segment's chunks in
// order with each head's P x N state held in MFMA accumulator registers, so the chunk-state
// tensor is never written to HBM. Per chunk of Q = 64 steps:
//   dt/decay  dt' = clamp(softplus(dt + dt_bias)) and the inclusive prefix sum of dt' * A_h
//             over the chunk with a 64-lane DPP scan, formed a chunk ahead by one wave per
//             head and read from LDS by the others.
//   staging   X, X * w with w_j = exp(acum_end - acum_j) dt'_j, and B go to LDS as bf16. C
//             goes to LDS too when two heads share it; with one head each wave keeps its 16
//             rows of C in registers.
//   Y_off     Y^T[p,i] = exp(acum_i) * sum_n S[p,n] C[i,n]              (MFMA, K = N)
//   Y_diag    S^T[j,i] = sum_n B[j,n] C[i,n]; mask j <= i; * exp(acum_i - acum_j) dt'_j;
//             Y^T[p,i] += sum_j X^T[p,j] S^T[j,i]                          (MFMA, K = N, Q)
//             with D_h added on the diagonal j == i, so Y^T is y^T
//   state     S = exp(acum_end) S + (X w)^T B                             (MFMA, K = Q)
// MFMA is v_mfma_f32_16x16x32_bf16 with fp32 accumulation.
//
// The internal chunk (Q = 64) is independent of the model's chunkLen: the chunked algorithm
// is exact for any chunk length. Long single sequences are cut into segments so that
// B*H*segments workgroups fill the chip: a state-only pass (ssd_state_kernel) gives each
// segment's local final state and total decay, a combine pass (ssd_seg_prefix) turns them into
// each segment's entering state, and the full pass (ssd_kernel) starts each segment from it.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "glue.hpp"
#include "ssd.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int Q = 64;     // internal chunk length
constexpr int P = 64;     // head dim handled by this kernel
constexpr int kTargetWG = 512;

struct SsdArgs {
    const void* x; long ldx;
    const float* dt; long lddt;
    const float* dt_bias; int softplus; float dt_min, dt_max;
    const float* A;
    const void* Bm; long ldb;
    const void* Cm; long ldc;
    const float* Dsk;
    float* y; long ldy;
    int B, L, H, G, N;
    int nchunks, nseg, chunks_per_seg;
    const float* h0;        // (B,H,P,N) or null
    float* hT;              // (B,H,P,N) or null
    float* seg_state;       // (B,H,nseg,P,N): local final state, then entering state
    float* seg_decay;       // (B,H,nseg): sum of dt' A over the segment
    int remap;              // XCD-aware workgroup order
};

__device__ __forceinline__ floatx4 mfma(bf16x8 a, bf16x8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ float ld1(const T* p);
template <>
__device__ __forceinline__ float ld1<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float ld1<__bf16>(const __bf16* p) { return (float)*p; }

__device__ __forceinline__ __bf16 hi_of(float v) { return (__bf16)v; }

// LDS tiles, all in natural row-major layout (rows = time steps j, or p for the state). The
// operands an MFMA needs with K = j (X^T, (X w)^T, B^T) are read with ds_read_b64_tr_b16:
// inside each 16-lane group, lane 4a+b receives element b of the 8-byte chunks addressed by
// lanes a, a+4, a+8, a+12. If lane m points at row j0 + m/4, column base + 4 (m % 4), lane L
// receives M[j0 .. j0+3][base + L]: four K-consecutive values of column base + L.
// Row pitches: X, X w and state^T P + 8, B N + 16 (bf16 elements). The b128 row reads of B
// are conflict-free at pitch 144; the transposed reads over rows j0 + 8 q4 (+4) meet 2-way
// bank conflicts at every pitch (SQ_LDS_BANK_CONFLICT). A layout without them (k-slot rows
// 4 q4 apart, pitches of 16 mod 32) ran no faster: LDS is not what bounds this kernel.
template <int NN, int HPW>
struct Smem {
    static constexpr int XP = P + 8;                   // X / Xw row pitch (bf16)
    static constexpr int BP = NN + 16;                 // B / C row pitch
    // 16-byte alignment lets the compiler use ds_read_b128 / ds_write_b128 for the 8-wide
    // bf16 rows (every pitch is a multiple of 8 elements). B and C belong to the group and
    // are staged once for the HPW heads of the workgroup; the other tiles are per head.
    alignas(16) __bf16 xw[HPW][Q][XP];                 // X * w_j   (j, p)
    alignas(16) __bf16 b[Q][BP];                       // B         (j, n)
    static constexpr bool CST = HPW > 1;               // C staged (shared by two heads)
    alignas(16) __bf16 c[CST ? Q : 1][BP];             // C   (i, n)
    alignas(16) __bf16 x[HPW][Q][XP];                  // X   (j, p)
    alignas(16) __bf16 s[HPW][NN][XP];                 // state^T (n, p)
    // two chunks' worth (the full pass scans a chunk ahead)
    alignas(16) float dv[2][HPW][Q];   // dt'_j
    alignas(16) float ac[2][HPW][Q];   // acum_j log2(e)
    alignas(16) float wj[2][HPW][Q];   // w_j = exp(acum_end - acum_j) dt'_j
    float ae[2][HPW];                  // acum_end
};

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// Transposed read: see Smem. `row0` is j0 for this lane's 16-lane group, `col0` the first of
// the 16 columns; returns M[j0..j0+3][col0 + (lane % 16)].
template <int PITCH>
__device__ __forceinline__ bf16x4 tr_read(const __bf16* base, int row0, int col0, int l16) {
    const __bf16* p = base + (row0 + (l16 >> 2)) * PITCH + col0 + 4 * (l16 & 3);
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
}

__device__ __forceinline__ bf16x8 cat(bf16x4 a, bf16x4 b) {
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Per-thread raw prefetch of one chunk. X (of the wave's head): wave w reads rows
// 16w .. 16w+15 as whole rows, XL lanes of 16 bytes (XE elements) per row and XR rows per
// load, so every load covers full 128-byte lines; lane t holds row 16w + XR k + t / XL,
// columns XE (t % XL) + 0 .. XE-1 of load k. B, and C when two heads share it (shared by the
// workgroup's heads): thread t of the workgroup reads rows t / (NN/8) + BR k, 8 elements at
// 8 (t % (NN/8)). dt: time step lane. With one head per workgroup each wave loads its own C
// rows as MFMA fragments instead (no staging).
template <int NN, bool FULL, int HPW>
struct Raw {
    static constexpr int KS = NN / 32;
    static constexpr int BL = NN / 8;                // lanes per B / C row
    static constexpr int BR = 256 * HPW / BL;        // B / C rows per pass
    static constexpr int BPASS = Q / BR;
    using v8 = bf16x8;
    static constexpr int XE = 8;                     // X elements per 16-byte load
    static constexpr int XL = P / XE;                // lanes per X row
    static constexpr int XR = 64 / XL;               // X rows per load
    static constexpr int XK = 16 / XR;               // X loads per wave
    v8 x[XK];
    v8 b[BPASS];
    v8 c[FULL && HPW > 1 ? BPASS : 1];
    float dt;
};

// Range-checked buffer access (raw buffer, stride 0, dword 3 = 0x00020000 on gfx9): a lane
// whose byte offset lies at or past num_records reads zeros and its stores are dropped.
// Every chunk gets descriptors whose num_records ends with its last valid time step, so the
// rows past the sequence end need no branches and every chunk issues the same memory
// instructions (the compiler can then count them exactly in its vmcnt waits).
using ssm::bload16;
using ssm::bload4;
using ssm::bstore16;
using ssm::rsrc;

// Inclusive prefix sum over the 64 lanes with DPP (row_shr inside rows of 16, then
// row_bcast:15 / row_bcast:31 across rows); no LDS traffic.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float add_dpp(float x) {
    const int y = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xf,
                                              true);
    return x + __builtin_bit_cast(float, y);
}

__device__ __forceinline__ float wave_prefix_sum(float v) {
    v = add_dpp<0x111, 0xf>(v);   // row_shr:1
    v = add_dpp<0x112, 0xf>(v);   // row_shr:2
    v = add_dpp<0x114, 0xf>(v);   // row_shr:4
    v = add_dpp<0x118, 0xf>(v);   // row_shr:8
    v = add_dpp<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    v = add_dpp<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
    return v;
}

// Value of the neighbouring lane (lane ^ 1, DPP quad_perm [1,0,3,2]) for every dword of v.
template <typename V>
__device__ __forceinline__ V swap_pair(V v) {
    static_assert(sizeof(V) == 16, "16-byte vectors");
    ssm::u32x4 u = __builtin_bit_cast(ssm::u32x4, v);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        u[i] = (unsigned)__builtin_amdgcn_mov_dpp((int)u[i], 0xB1, 0xf, 0xf, true);
    return __builtin_bit_cast(V, u);
}

template <typename V>
__device__ __forceinline__ V vzero() {
    V v;
    __builtin_memset(&v, 0, sizeof v);
    return v;
}

// Launch shape: HPW heads of one group per workgroup (4 waves per head). When heads pair up
// in a group, two heads per workgroup (8 waves, one workgroup per CU): B and C are loaded and
// staged once for both heads, which halves their share of the memory instructions.
template <int NN, int HPW>
__global__ __launch_bounds__(256 * HPW, HPW > 1 ? 1 : 2) void ssd_kernel(SsdArgs a) {
    using TIN = __bf16;
    __shared__ __attribute__((aligned(16))) Smem<NN, HPW> sm;
    using SM = Smem<NN, HPW>;
    constexpr int NB = NN / 16;   // state n-blocks per wave
    constexpr int KS = NN / 32;   // k-steps over n
    using RW = Raw<NN, true, HPW>;
    constexpr bool CST = SM::CST;       // C staged in LDS (two heads) or loaded per wave

    int wg = blockIdx.x;
    if (a.remap) {
        const int per = gridDim.x / 8;
        wg = (blockIdx.x % 8) * per + blockIdx.x / 8;
    }
    // segment-major order: the head groups of one (batch, segment) are adjacent, so after the
    // XCD remap they run on the same XCD and read that segment's B and C through one L2
    const int HW = a.H / HPW;   // workgroups per (batch, segment)
    const int seg = wg / (a.B * HW);
    const int bhw = wg % (a.B * HW);
    const int b = bhw / HW;
    // w is wave-uniform: readfirstlane lets the compiler keep it (and the j-block loop
    // bounds derived from it) in scalar registers. Wave w works on head hw = w / 4 of the
    // workgroup as its wave wl: w % 4 for the first head, 3 - w % 4 for the second. Waves w and
    // w + 4 share a SIMD, and Y_diag grows with wl, so each SIMD gets one light and one heavy
    // wave.
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hw = w >> 2, wl = (hw & 1) ? 3 - (w & 3) : (w & 3);
    const int h = HPW * (bhw % HW) + hw;
    const int bh = b * a.H + h;
    const int g = h / (a.H / a.G);
    const int l16 = lane & 15, q4 = lane >> 4;
    const int ic = 16 * wl + l16;       // this lane's output row in the chunk
    const int br = tid / RW::BL, bc = 8 * (tid % RW::BL);      // B / C staging row / column

    const float Ah = a.A[h];
    const float dtb = a.dt_bias ? a.dt_bias[h] : 0.f;
    const float Dh = a.Dsk ? a.Dsk[h] : 0.f;

    const int c_begin = seg * a.chunks_per_seg;
    const int c_end = min(c_begin + a.chunks_per_seg, a.nchunks);

    // Chunk c starts at row b*L + c*Q of every (B, L, ...) tensor; per-lane byte offsets
    // inside a chunk are the same for every chunk (the host checks that Q rows of every
    // tensor span less than 2^31 bytes).
    constexpr unsigned SZ = sizeof(TIN);
    const long brow = (long)b * a.L;
    const TIN* x0 = reinterpret_cast<const TIN*>(a.x) + brow * a.ldx + (long)h * P;
    const TIN* b0 = reinterpret_cast<const TIN*>(a.Bm) + brow * a.ldb + (long)g * a.N;
    const TIN* cm0 = reinterpret_cast<const TIN*>(a.Cm) + brow * a.ldc + (long)g * a.N;
    const float* d0 = a.dt + brow * a.lddt + h;
    const int xr = lane / RW::XL, xc = RW::XE * (lane % RW::XL);   // X row in a load / column
    const unsigned ox = (unsigned)((16 * wl + xr) * a.ldx + xc) * SZ;
    const unsigned oxk = (unsigned)(RW::XR * a.ldx) * SZ;
    const unsigned ob = (unsigned)(br * a.ldb + bc) * SZ;
    const unsigned obk = (unsigned)(RW::BR * a.ldb) * SZ;
    const unsigned occ = (unsigned)(br * a.ldc + bc) * SZ;
    const unsigned occk = (unsigned)(RW::BR * a.ldc) * SZ;
    const unsigned od = (unsigned)(lane * a.lddt) * 4u;
    // Lanes l16 = 2r and 2r + 1 share the 128-byte lines of rows 16wl + 2r and 16wl + 2r + 1:
    // the y store (and, without C staging, the C load) (h, sel) of lane (l16, q4) covers row
    // 16wl + (l16 & ~1) + sel at byte 128 h + 64 (l16 & 1) + 16 q4 of the row, so each such
    // instruction moves whole lines of 8 rows. A DPP swap between the two lanes puts every
    // value where the MFMA layout has it.
    const int podd = l16 & 1;
    const unsigned oc2 = (unsigned)((16 * wl + l16 - podd) * a.ldc + 32 * podd + 8 * q4) * SZ;
    // rows of chunk c that exist; 0 past the segment, so a prefetch there reads nothing
    auto rows_of = [&](int c) { return c < c_end ? min(Q, a.L - c * Q) : 0; };
    auto span = [](int qv, long ld, int width, unsigned esz) {
        return qv > 0 ? (unsigned)(((long)(qv - 1) * ld + width) * esz) : 0u;
    };

    RW raw;
    using v8 = typename RW::v8;
    // x, B (, C) of chunk c and dt of chunk cd (the full pass reads dt one chunk further
    // ahead: its scan runs a chunk early, below)
    auto load_raw = [&](int c, int cd) {
        const int qv = rows_of(c);
        const long r0 = (long)c * Q;
        // dt: one strided 4-byte value per step (a cache line per lane); only the wave that
        // scans fetches it, the others get an empty descriptor (no traffic)
        const auto rd = rsrc(d0 + (long)cd * Q * a.lddt, wl != 0 ? 0u : span(rows_of(cd), a.lddt, 1, 4));
        const auto rx = rsrc(x0 + r0 * a.ldx, span(qv, a.ldx, P, SZ));
        const auto rb = rsrc(b0 + r0 * a.ldb, span(qv, a.ldb, NN, SZ));
        raw.dt = bload4(rd, od);
        // x is read by this head only: streaming loads; B (and C) serve every head of the
        // group on this XCD and stay ordinary, so the other heads find them in L2
#pragma unroll
        for (int k = 0; k < RW::XK; ++k) raw.x[k] = ssm::bload16_nt<v8>(rx, ox + k * oxk);
#pragma unroll
        for (int k = 0; k < RW::BPASS; ++k) raw.b[k] = bload16<v8>(rb, ob + k * obk);
        if constexpr (CST) {
            const auto rc = rsrc(cm0 + r0 * a.ldc, span(qv, a.ldc, NN, SZ));
#pragma unroll
            for (int k = 0; k < RW::BPASS; ++k) raw.c[k] = bload16<v8>(rc, occ + k * occk);
        }
    };
    // Without C staging: C rows of the wave's strip, row ic, n = 32ks + 8q4 + 0..7 (MFMA
    // B-operand fragments), prefetched after their last use in the previous chunk
    v8 craw[!CST ? KS : 1];
    auto load_c = [&](int c) {
        if constexpr (!CST) {
            const int qv = rows_of(c);
            const auto rc = rsrc(cm0 + (long)c * Q * a.ldc, span(qv, a.ldc, NN, SZ));
            // craw[2h + sel]: row 16wl + (l16 & ~1) + sel, n = 64h + 32 (l16 & 1) + 8 q4 + 0..7
#pragma unroll
            for (int hh = 0; hh < KS / 2; ++hh)
#pragma unroll
                for (int sel = 0; sel < 2; ++sel)
                    craw[2 * hh + sel] =
                        bload16<v8>(rc, oc2 + (unsigned)(sel * a.ldc * SZ) + 128u * hh);
        }
    };
    // 8 elements of B or C to LDS
    auto stage8 = [&](__bf16 (*tile)[SM::BP], int j, const v8& src) {
        *reinterpret_cast<bf16x8*>(&tile[j][bc]) = src;
    };

    // ---- entering state -> accumulators (wave wl: rows p = 16wl + 4*q4 + r, cols 16nb + l16)
    const float* init = nullptr;
    if (a.nseg > 1) init = a.seg_state + ((long)bh * a.nseg + seg) * P * NN;
    else if (a.h0) init = a.h0 + (long)bh * P * NN;
    floatx4 S[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            S[nb][r] = init ? init[(long)(16 * wl + 4 * q4 + r) * NN + 16 * nb + l16] : 0.f;
    bool state_live = init != nullptr;

    // The accumulators hold S[p = 16wl + 4q4 + r][n = 16nb + l16] for r = 0..3: four
    // consecutive p of one n, i.e. one 8-byte run of the state^T tile.
    auto write_state_lds = [&]() {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            bf16x4 hv;
#pragma unroll
            for (int r = 0; r < 4; ++r) hv[r] = hi_of(S[nb][r]);
            *reinterpret_cast<bf16x4*>(&sm.s[hw][16 * nb + l16][16 * wl + 4 * q4]) = hv;
        }
    };
    if (state_live) write_state_lds();
    // dt' of chunk cc (0 past the segment), acum in log2 units, the weights w_j and acum_end of
    // the wave's head into LDS buffer bf (lane = time step)
    auto scan_put = [&](int cc, float raw_dt, int bf) {
        const int qv = rows_of(cc);
        float dv = raw_dt + dtb;
        if (a.softplus) dv = ssm::softplus_fast(dv);
        dv = lane < qv ? fminf(fmaxf(dv, a.dt_min), a.dt_max) : 0.f;
        const float sc = wave_prefix_sum(dv * Ah);
        const float ae = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), 63));
        // decay weight exp(acum_i - acum_j) dt'_j = exp2(ac_i - ac_j) dt'_j: dt' keeps its
        // sign (softplus off with no lower clamp allows dt' < 0)
        sm.dv[bf][hw][lane] = dv;
        sm.ac[bf][hw][lane] = sc * ssm::kLog2e;
        sm.wj[bf][hw][lane] = ssm::ex2((ae - sc) * ssm::kLog2e) * dv;
        if (lane == 0) sm.ae[bf][hw] = ae;
    };
    // the first chunk's scan (in the loop, each head's wave with the lightest Y_diag scans the
    // next chunk while the others work); dt of the second chunk comes with the inputs
    if (wl == 0) {
        const auto rd0 = rsrc(d0 + (long)c_begin * Q * a.lddt, span(rows_of(c_begin), a.lddt, 1, 4));
        scan_put(c_begin, bload4(rd0, od), c_begin & 1);
    }
    __syncthreads();
    load_raw(c_begin, c_begin + 1);
    load_c(c_begin);
    {
        // Four stores into an empty range (dropped by the range check) make the memory
        // instructions in flight at loop entry match the back edge (the prefetches, then the
        // four y stores), so the wait for a prefetch never includes the previous chunk's stores.
        const auto none = rsrc(a.y, 0u);
#pragma unroll
        for (int pb = 0; pb < P / 16; ++pb) bstore16(make_float4(0.f, 0.f, 0.f, 0.f), none, 64u * pb);
    }

    for (int c = c_begin; c < c_end; ++c) {
        const int t0 = c * Q;
        const int qv = min(Q, a.L - t0);
        const long row0 = (long)b * a.L + t0;

        const int buf = c & 1;
        // dt', the prefix of dt' * A and w_j of this chunk were formed a chunk earlier
        const float acend = sm.ae[buf][hw];

        // ---- stage X and X w (rows of the X prefetch)
#pragma unroll
        for (int k = 0; k < RW::XK; ++k) {
            constexpr int E = RW::XE;
            const int j = 16 * wl + RW::XR * k + xr;
            const float wj = sm.wj[buf][hw][j];
            bf16x8 wh;
#pragma unroll
            for (int e = 0; e < E; ++e) wh[e] = hi_of((float)raw.x[k][e] * wj);
            *reinterpret_cast<bf16x8*>(&sm.xw[hw][j][xc]) = wh;
            *reinterpret_cast<bf16x8*>(&sm.x[hw][j][xc]) = raw.x[k];
        }
        // ---- stage B and C (shared by the workgroup's heads)
#pragma unroll
        for (int k = 0; k < RW::BPASS; ++k) {
            stage8(sm.b, br + RW::BR * k, raw.b[k]);
            if constexpr (CST) stage8(sm.c, br + RW::BR * k, raw.c[k]);
        }
        // ---- C rows of this wave's strip as MFMA fragments: row ic, n = 32ks + 8q4 + 0..7
        // (from registers here without C staging, from LDS after the barrier with it)
        bf16x8 cfh[KS];
        if constexpr (!CST) {
            // fragment ks = 2h + e of row ic: the own load (h, sel = l16 & 1) holds e = l16 & 1,
            // the neighbour's load (h, sel = l16 & 1) the other one
#pragma unroll
            for (int hh = 0; hh < KS / 2; ++hh) {
                const bf16x8 s0 = swap_pair(craw[2 * hh]);
                const bf16x8 s1 = swap_pair(craw[2 * hh + 1]);
                cfh[2 * hh] = podd ? s1 : craw[2 * hh];
                cfh[2 * hh + 1] = podd ? craw[2 * hh + 1] : s0;
            }
        }
        __syncthreads();   // staging (and the state LDS copy) visible to every wave

        // ---- the next chunk's raw inputs are in flight while this one computes (a chunk past
        // the segment has an empty range: the loads return zeros without touching memory)
        const float dnext = raw.dt;   // dt of chunk c + 1
        load_raw(c + 1, c + 2);

        {
            if constexpr (CST) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    cfh[ks] = *reinterpret_cast<const bf16x8*>(&sm.c[ic][32 * ks + 8 * q4]);
            }
            const float aci = sm.ac[buf][hw][ic];
            floatx4 Y[P / 16];
#pragma unroll
            for (int pb = 0; pb < P / 16; ++pb) Y[pb] = floatx4{0.f, 0.f, 0.f, 0.f};

            // ---- Y_off = exp(acum_i) * S C^T
            if (state_live) {
#pragma unroll
                for (int pb = 0; pb < P / 16; ++pb) {
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        // S[p = 16pb + l16][n = 32ks + 8q4 + 0..7] from the state^T tile
                        const int n0 = 32 * ks + 8 * q4;
                        const bf16x8 ah = cat(tr_read<SM::XP>(&sm.s[hw][0][0], n0, 16 * pb, l16),
                                              tr_read<SM::XP>(&sm.s[hw][0][0], n0 + 4, 16 * pb, l16));
                        Y[pb] = mfma(ah, cfh[ks], Y[pb]);
                    }
                }
                const float e = ssm::ex2(aci);
#pragma unroll
                for (int pb = 0; pb < P / 16; ++pb) Y[pb] *= e;
            }

            // ---- Y_diag: wave wl's rows i = 16wl + l16 need the j-blocks 0..wl. The body is
            // unrolled per wave (switch on the wave-uniform wl) so the independent C B^T chains
            // of the j-blocks interleave. D_h x_i rides on the diagonal (j == i) of the decay
            // matrix: y_i = sum_j (L[i,j] + D_h [i == j]) x_j.
            auto y_diag = [&](auto wc) {
                constexpr int W = decltype(wc)::value;
                floatx4 st[W + 1];
#pragma unroll
                for (int jb = 0; jb <= W; ++jb) st[jb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int jb = 0; jb <= W; ++jb) {
                        const bf16x8 bh_ = *reinterpret_cast<const bf16x8*>(
                            &sm.b[16 * jb + l16][32 * ks + 8 * q4]);
                        st[jb] = mfma(bh_, cfh[ks], st[jb]);
                    }
                // S^T[j, i] * exp(acum_i - acum_j) dt'_j for this lane's rows j = 16jb + 4q4 + r;
                // below the diagonal block every j < i, on it j > i is masked by a select (the
                // dropped exp may overflow)
                float sv[2 * (W / 2 + 1)][4];
#pragma unroll
                for (int jb = 0; jb < 2 * (W / 2 + 1); ++jb) {
                    if (jb > W) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) sv[jb][r] = 0.f;
                        continue;
                    }
                    const float4 aj = *reinterpret_cast<const float4*>(&sm.ac[buf][hw][16 * jb + 4 * q4]);
                    const float4 dj = *reinterpret_cast<const float4*>(&sm.dv[buf][hw][16 * jb + 4 * q4]);
                    const float ajr[4] = {aj.x, aj.y, aj.z, aj.w};
                    const float djr[4] = {dj.x, dj.y, dj.z, dj.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float f = st[jb][r] * (ssm::ex2(aci - ajr[r]) * djr[r]);
                        if (jb < W) {
                            sv[jb][r] = f;
                        } else {
                            const int dj = 4 * q4 + r;   // j - 16wl
                            sv[jb][r] = dj < l16 ? f : (dj == l16 ? f + Dh : 0.f);
                        }
                    }
                }
                // X^T fragment: k-slots 0..3 <-> j = 32 jb2 + 4 q4 + 0..3, 4..7 <-> +16
#pragma unroll
                for (int jb2 = 0; jb2 <= W / 2; ++jb2) {
                    bf16x8 sfh;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        sfh[r] = hi_of(sv[2 * jb2][r]);
                        sfh[4 + r] = hi_of(sv[2 * jb2 + 1][r]);
                    }
#pragma unroll
                    for (int pb = 0; pb < P / 16; ++pb) {
                        const bf16x8 xh = cat(tr_read<SM::XP>(&sm.x[hw][0][0], 32 * jb2 + 4 * q4, 16 * pb, l16),
                                              tr_read<SM::XP>(&sm.x[hw][0][0], 32 * jb2 + 16 + 4 * q4, 16 * pb, l16));
                        Y[pb] = mfma(xh, sfh, Y[pb]);
                    }
                }
            };
            switch (wl) {
                case 0: y_diag(std::integral_constant<int, 0>{}); break;
                case 1: y_diag(std::integral_constant<int, 1>{}); break;
                case 2: y_diag(std::integral_constant<int, 2>{}); break;
                default: y_diag(std::integral_constant<int, 3>{}); break;
            }
            // the lightest wave scans chunk c + 1 into the other buffers (the last reads of
            // those, chunk c - 1's, came before this chunk's first barrier)
            if (wl == 0) scan_put(c + 1, dnext, buf ^ 1);

            // ---- the next chunk's C fragments (the last use of this chunk's was Y_diag)
            load_c(c + 1);

            // ---- y: Y[pb] holds row ic, p = 16pb + 4q4 + 0..3; store (h, sel) writes p-half h
            // of row 16wl + (l16 & ~1) + sel. Rows past the sequence end fall outside the
            // descriptor and are dropped.
            {
                const auto ry = rsrc(a.y + (row0 * a.ldy + (long)h * P), span(qv, a.ldy, P, 4));
                const unsigned oy = (unsigned)((16 * wl + l16 - podd) * a.ldy + 16 * podd + 4 * q4) * 4u;
#pragma unroll
                for (int hh = 0; hh < P / 32; ++hh) {
                    const floatx4 s0 = swap_pair(Y[2 * hh]), s1 = swap_pair(Y[2 * hh + 1]);
                    const floatx4 v0 = podd ? s1 : Y[2 * hh];        // row 16wl + (l16 & ~1)
                    const floatx4 v1 = podd ? Y[2 * hh + 1] : s0;    // row 16wl + (l16 & ~1) + 1
                    // y streams out (read by the next launch only)
                    ssm::bstore16_nt(make_float4(v0[0], v0[1], v0[2], v0[3]), ry, oy + 128u * hh);
                    ssm::bstore16_nt(make_float4(v1[0], v1[1], v1[2], v1[3]), ry,
                                     oy + (unsigned)(a.ldy * 4) + 128u * hh);
                }
            }
        }

        // ---- state: S = exp(acum_end) S + (X w)^T B   (k-slots j = 32ks + 8q4 + 0..7)
        {
            const float e = ssm::ex2(acend * ssm::kLog2e);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) S[nb] *= e;
#pragma unroll
            for (int ks = 0; ks < Q / 32; ++ks) {
                const int j0 = 32 * ks + 8 * q4;
                const bf16x8 xh = cat(tr_read<SM::XP>(&sm.xw[hw][0][0], j0, 16 * wl, l16),
                                      tr_read<SM::XP>(&sm.xw[hw][0][0], j0 + 4, 16 * wl, l16));
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const bf16x8 bh_ = cat(tr_read<SM::BP>(&sm.b[0][0], j0, 16 * nb, l16),
                                           tr_read<SM::BP>(&sm.b[0][0], j0 + 4, 16 * nb, l16));
                    S[nb] = mfma(xh, bh_, S[nb]);
                }
            }
        }
        state_live = true;
        __syncthreads();   // every wave is done reading this chunk's LDS
        if (c + 1 < c_end) write_state_lds();
    }

    // ---- the final state (last segment)
    if (a.hT && seg == a.nseg - 1) {
        float* out = a.hT + (long)bh * P * NN;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) out[(long)(16 * wl + 4 * q4 + r) * NN + 16 * nb + l16] = S[nb][r];
    }
}

// State-only pass of the segmented mode (long sequences with few batch x heads): a workgroup
// reads x, B and dt of one (batch, segment) and HPW heads of one group once and returns each
// head's local final state of the segment (from a zero state) and its total decay sum(dt' A).
// B is staged once for the HPW heads. Per chunk: each head's wave 0 scans the next chunk's dt
// (dt', its prefix sum of dt' A, w_j = exp(acum_end - acum_j) dt'_j) into LDS; every wave
// stages X w (and its share of B) into LDS; one barrier; then S = exp(acum_end) S + (X w)^T B
// (wave 4 hw + wl: head hw, state rows p = 16 wl .. 16 wl + 15). dt is one strided 4-byte value
// per step, a cache line per lane, so only the scanning waves fetch it (the others' descriptor
// is empty). The loads run kStateDepth
// chunks ahead in a ring of register sets (the chunk loop is unrolled by the ring size, so each
// set keeps fixed registers), and the LDS tiles are double-buffered: a wave writes a buffer two
// chunks after it was read, with a barrier between.
constexpr int kStateDepth = 4;

template <int NN, int HPW>
__global__ __launch_bounds__(256 * HPW, HPW > 1 ? 1 : 2) void ssd_state_kernel(SsdArgs a) {
    using TIN = __bf16;
    using RW = Raw<NN, false, HPW>;
    using v8 = typename RW::v8;
    constexpr int XP = P + 8, BP = NN + 16, NB = NN / 16, DEPTH = kStateDepth;
    static_assert(DEPTH % 2 == 0, "the LDS buffer of ring slot k is k % 2");
    __shared__ __attribute__((aligned(16))) __bf16 sxw[2][HPW][Q][XP];   // X w_j  (j, p)
    __shared__ __attribute__((aligned(16))) __bf16 sb[2][Q][BP];         // B      (j, n)
    __shared__ float sw[2][HPW][Q];    // w_j = exp(acum_end - acum_j) dt'_j
    __shared__ float sae[2][HPW];      // acum_end

    int wg = blockIdx.x;
    if (a.remap) {
        const int per = gridDim.x / 8;
        wg = (blockIdx.x % 8) * per + blockIdx.x / 8;
    }
    // segment-major: the head groups of one (batch, segment) are adjacent and share B through
    // one L2. Wave w works on head hw = w / 4 of the workgroup, state rows 16 wl .. 16 wl + 15.
    const int HW = a.H / HPW;
    const int seg = wg / (a.B * HW);
    const int bhw = wg % (a.B * HW);
    const int b = bhw / HW;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hw = w >> 2, wl = w & 3;
    const int h = HPW * (bhw % HW) + hw;
    const int bh = b * a.H + h;
    const int g = h / (a.H / a.G);
    const int l16 = lane & 15, q4 = lane >> 4;
    const int br = tid / RW::BL, bc = 8 * (tid % RW::BL);
    const float Ah = a.A[h];
    const float dtb = a.dt_bias ? a.dt_bias[h] : 0.f;
    const int c_begin = seg * a.chunks_per_seg;
    const int c_end = min(c_begin + a.chunks_per_seg, a.nchunks);

    constexpr unsigned SZ = sizeof(TIN);
    const long brow = (long)b * a.L;
    const TIN* x0 = reinterpret_cast<const TIN*>(a.x) + brow * a.ldx + (long)h * P;
    const TIN* b0 = reinterpret_cast<const TIN*>(a.Bm) + brow * a.ldb + (long)g * a.N;
    const float* d0 = a.dt + brow * a.lddt + h;
    const int xr = lane / RW::XL, xc = RW::XE * (lane % RW::XL);
    const unsigned ox = (unsigned)((16 * wl + xr) * a.ldx + xc) * SZ;
    const unsigned oxk = (unsigned)(RW::XR * a.ldx) * SZ;
    const unsigned ob = (unsigned)(br * a.ldb + bc) * SZ;
    const unsigned obk = (unsigned)(RW::BR * a.ldb) * SZ;
    const unsigned od = (unsigned)(lane * a.lddt) * 4u;
    auto rows_of = [&](int c) { return c < c_end ? min(Q, a.L - c * Q) : 0; };
    auto span = [](int qv, long ld, int width, unsigned esz) {
        return qv > 0 ? (unsigned)(((long)(qv - 1) * ld + width) * esz) : 0u;
    };
    // x, B and dt of chunk c (a chunk past the segment has an empty range: zeros, no traffic)
    auto load_raw = [&](RW& r, int c) {
        const int qv = rows_of(c);
        const long r0 = (long)c * Q;
        // dt: one strided 4-byte value per step (a cache line per lane), so only each head's
        // wave 0, which scans, fetches it; the other waves' descriptor is empty (no traffic)
        const auto rd = rsrc(d0 + r0 * a.lddt, wl == 0 ? span(qv, a.lddt, 1, 4) : 0u);
        const auto rx = rsrc(x0 + r0 * a.ldx, span(qv, a.ldx, P, SZ));
        const auto rb = rsrc(b0 + r0 * a.ldb, span(qv, a.ldb, NN, SZ));
        r.dt = bload4(rd, od);
        // streaming x loads, as in the full pass (with ordinary loads here, the full pass's
        // streaming reads of the same x measured slower: 257.6 against 232.0 us at cfg5)
#pragma unroll
        for (int k = 0; k < RW::XK; ++k) r.x[k] = ssm::bload16_nt<v8>(rx, ox + k * oxk);
#pragma unroll
        for (int k = 0; k < RW::BPASS; ++k) r.b[k] = bload16<v8>(rb, ob + k * obk);
    };

    RW raw[DEPTH];
#pragma unroll
    for (int k = 0; k < DEPTH; ++k) {
        load_raw(raw[k], c_begin + k);
        __builtin_amdgcn_sched_barrier(0);
    }

    floatx4 S[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) S[nb] = floatx4{0.f, 0.f, 0.f, 0.f};
    float decay_sum = 0.f;   // each head's wave 0
    // each head's wave 0: dt' of chunk cc (0 past the segment), its prefix sum of dt' A, the
    // weights w_j and acum_end into buffer bf (lane = step)
    auto scan_put = [&](int cc, float raw_dt, int bf) {
        const int qv = rows_of(cc);
        float dv = raw_dt + dtb;
        if (a.softplus) dv = ssm::softplus_sel(dv);
        dv = lane < qv ? fminf(fmaxf(dv, a.dt_min), a.dt_max) : 0.f;
        const float sc = wave_prefix_sum(dv * Ah);
        const float ae = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), 63));
        sw[bf][hw][lane] = ssm::ex2((ae - sc) * ssm::kLog2e) * dv;
        if (lane == 0) sae[bf][hw] = ae;
        decay_sum += ae;
    };
    if (wl == 0) scan_put(c_begin, raw[0].dt, 0);
    __syncthreads();

    // Whole groups of DEPTH chunks with no exit inside a group, so that the loads in flight at
    // the loop head are the same on entry and on the back edge and the compiler's vmcnt waits
    // stay exact. A chunk past the segment reads zeros (dt' = 0, w = 0, decay 1): it leaves
    // the state and the decay sum unchanged.
    for (int c0 = c_begin; c0 < c_end; c0 += DEPTH) {
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) {
            const int c = c0 + k;
            const int buf = k & 1;
            // wave 0 scans the next chunk (its dt is the first load of the next ring slot) into
            // the other buffer, which every wave last read before the previous barrier
            if (wl == 0) scan_put(c + 1, raw[(k + 1) % DEPTH].dt, buf ^ 1);
            const float acend = sae[buf][hw];
#pragma unroll
            for (int kx = 0; kx < RW::XK; ++kx) {
                const int j = 16 * wl + RW::XR * kx + xr;
                const float wj = sw[buf][hw][j];
                bf16x8 wh;
#pragma unroll
                for (int e = 0; e < RW::XE; ++e) wh[e] = hi_of((float)raw[k].x[kx][e] * wj);
                *reinterpret_cast<bf16x8*>(&sxw[buf][hw][j][xc]) = wh;
            }
#pragma unroll
            for (int kb = 0; kb < RW::BPASS; ++kb)
                *reinterpret_cast<bf16x8*>(&sb[buf][br + RW::BR * kb][bc]) = raw[k].b[kb];
            load_raw(raw[k], c + DEPTH);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();

            const float e = ssm::ex2(acend * ssm::kLog2e);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) S[nb] *= e;
#pragma unroll
            for (int ks = 0; ks < Q / 32; ++ks) {
                const int j0 = 32 * ks + 8 * q4;
                const bf16x8 xh = cat(tr_read<XP>(&sxw[buf][hw][0][0], j0, 16 * wl, l16),
                                      tr_read<XP>(&sxw[buf][hw][0][0], j0 + 4, 16 * wl, l16));
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const bf16x8 bv = cat(tr_read<BP>(&sb[buf][0][0], j0, 16 * nb, l16),
                                          tr_read<BP>(&sb[buf][0][0], j0 + 4, 16 * nb, l16));
                    S[nb] = mfma(xh, bv, S[nb]);
                }
            }
        }
    }

    float* out = a.seg_state + ((long)bh * a.nseg + seg) * P * NN;
    if (wl == 0 && lane == 0) a.seg_decay[(long)bh * a.nseg + seg] = decay_sum;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) out[(long)(16 * wl + 4 * q4 + r) * NN + 16 * nb + l16] = S[nb][r];
}

// Segment entering states: slot[s] <- carry; carry = exp(decay[s]) carry + local[s].
__global__ void ssd_seg_prefix(SsdArgs a, int PN) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)a.B * a.H * PN) return;
    ssm::seg_prefix_elem(a.seg_state, a.seg_decay, a.h0, a.nseg, PN, i / PN, (int)(i % PN),
                         ssm::kLog2e);
}

template <int NN, int HPW>
ssm_status launch_ssd(SsdArgs& a, hipStream_t st) {
    if (a.nseg > 1) {
        // the state-only pass (ssd_state_kernel, HPW heads per workgroup). The last segment's
        // local state is never combined (the full pass produces the final state), so only the
        // first nseg - 1 segments run (the order is segment-major: they are the first
        // B*(H/HPW)*(nseg-1) workgroups).
        SsdArgs s1 = a;
        const int nwg1 = a.B * (a.H / HPW) * (a.nseg - 1);
        s1.remap = (nwg1 % 8 == 0) ? 1 : 0;
        ssd_state_kernel<NN, HPW><<<nwg1, 256 * HPW, 0, st>>>(s1);
        ssm_status e = ssm::check_launch("ssd_state_pass");
        if (e != SSM_OK) return e;
        const long n = (long)a.B * a.H * P * NN;
        ssd_seg_prefix<<<(unsigned)ssm::cdiv(n, 256), 256, 0, st>>>(a, P * NN);
        e = ssm::check_launch("ssd_seg_prefix");
        if (e != SSM_OK) return e;
    }
    const int nwg = a.B * (a.H / HPW) * a.nseg;
    a.remap = (nwg % 8 == 0) ? 1 : 0;
    ssd_kernel<NN, HPW><<<nwg, 256 * HPW, 0, st>>>(a);
    return ssm::check_launch("ssd_chunk_scan");
}

void plan(int B, int L, int H, int& nchunks, int& nseg, int& per) {
    nchunks = (int)ssm::cdiv(L, Q);
    const long bh = (long)B * H;
    long s = ssm::cdiv(kTargetWG, bh > 0 ? bh : 1);
    if (s > nchunks) s = nchunks;
    if (s < 1) s = 1;
    per = (int)ssm::cdiv(nchunks, s);
    nseg = (int)ssm::cdiv(nchunks, per);
}

// ---------------------------------------------------------------- one-token update (K7)
// HBM-bound: the (B,H,P,N) state is read and written once. Work split: a workgroup owns R
// passes of RPP = 256 / LPR rows of one (b, h) state (LPR = N / 4 lanes per row, one float4
// each), so the grid is B*H*ceil(P / (RPP*R)) workgroups of straight-line code, each thread
// with R state loads in flight; y[p] = C . h[p,:] + D x[p] is reduced over the row's lanes.
// The state goes through non-temporal loads and stores: it is touched once per step and not
// again before the other layers' states have streamed through the caches, and keeping it out
// of L2 and the MALL measured 13% faster (22.8 against 26.1 us at 64 x 32 x 64 x 128).
//
// GATED: y = (C.h + D x) * silu(z) * gn (the gated RMSNorm's element-wise part), stored in
// fragment order for the out_proj (frag_off, K = H * P), and the workgroup's sum of
// ((C.h + D x) silu(z))^2 over its rows into ssq[blockIdx.x] (a row's partial sums are
// contiguous: blockIdx.x = (b H + h) * blocks_per_head + block). z and gn are fetched with
// the state, so that no load waits behind the reduction.
//
// FULL: Pd is a whole number of workgroup row blocks (RPP * R), so no row needs a bound check;
// with the checks, each guarded load sat behind its own branch and the compiler waited for
// it before issuing the next, serialising the state loads.
template <int LPR, int R, bool GATED, bool FULL>
__global__ __launch_bounds__(256) void m2_update_kernel(
    const float* __restrict__ x, long ldx, const float* __restrict__ dt, long lddt,
    const float* __restrict__ dt_bias, int softplus, float dt_min, float dt_max,
    const float* __restrict__ A, const float* __restrict__ Bm, long ldb,
    const float* __restrict__ Cm, long ldc, const float* __restrict__ Dsk,
    const float* __restrict__ z, long ldz, const float* __restrict__ gn,
    float* __restrict__ ssq, float* __restrict__ y, long ldy,
    float* __restrict__ hs, int H, int Pd, int G, int N, int blocks_per_head) {
    constexpr int RPP = 256 / LPR;
    __shared__ float sq[GATED ? RPP * R : 1];
    const int tid = threadIdx.x;
    const int c4 = tid % LPR;            // float4 column
    const int rsub = tid / LPR;
    const int bh = blockIdx.x / blocks_per_head;
    const int p0 = (blockIdx.x % blocks_per_head) * RPP * R + rsub;
    const int h = bh % H, b = bh / H, g = h / (H / G);
    float* hb = hs + (long)bh * Pd * N;

    float4 v[R];
    float xp[R], zg[R], gg[R];
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int p = p0 + k * RPP;
        if (FULL || p < Pd) {
            const float* src = hb + (long)p * N + 4 * c4;
            v[k] = make_float4(__builtin_nontemporal_load(src), __builtin_nontemporal_load(src + 1),
                               __builtin_nontemporal_load(src + 2), __builtin_nontemporal_load(src + 3));
            xp[k] = x[(long)b * ldx + (long)h * Pd + p];
            if (GATED) {
                zg[k] = z[(long)b * ldz + (long)h * Pd + p];
                gg[k] = gn[(long)h * Pd + p];
            }
        }
    }
    const float4 bv = *reinterpret_cast<const float4*>(Bm + (long)b * ldb + (long)g * N + 4 * c4);
    const float4 cv = *reinterpret_cast<const float4*>(Cm + (long)b * ldc + (long)g * N + 4 * c4);
    float dl = dt[(long)b * lddt + h] + (dt_bias ? dt_bias[h] : 0.f);
    if (softplus) dl = ssm::softplus(dl);
    dl = fminf(fmaxf(dl, dt_min), dt_max);
    const float dA = ssm::ex2(dl * A[h] * ssm::kLog2e);
    const float Dh = Dsk ? Dsk[h] : 0.f;
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int p = p0 + k * RPP;
        if (!FULL && p >= Pd) {
            if (GATED && c4 == 0) sq[k * RPP + rsub] = 0.f;
            continue;
        }
        const float dx = dl * xp[k];
        float4 u = v[k];
        u.x = fmaf(dA, u.x, dx * bv.x);
        u.y = fmaf(dA, u.y, dx * bv.y);
        u.z = fmaf(dA, u.z, dx * bv.z);
        u.w = fmaf(dA, u.w, dx * bv.w);
        float* dst = hb + (long)p * N + 4 * c4;
        __builtin_nontemporal_store(u.x, dst);
        __builtin_nontemporal_store(u.y, dst + 1);
        __builtin_nontemporal_store(u.z, dst + 2);
        __builtin_nontemporal_store(u.w, dst + 3);
        float acc = u.x * cv.x + u.y * cv.y + u.z * cv.z + u.w * cv.w;
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, LPR);
        if (c4 == 0) {
            acc = fmaf(Dh, xp[k], acc);
            if (GATED) {
                acc *= ssm::silu(zg[k]);
                sq[k * RPP + rsub] = acc * acc;
                y[ssm::frag_off(b, h * Pd + p, H * Pd / 16)] = acc * gg[k];
            } else {
                if (z) acc *= ssm::silu(z[(long)b * ldz + (long)h * Pd + p]);
                y[(long)b * ldy + (long)h * Pd + p] = acc;
            }
        }
    }
    if constexpr (GATED) {
        // the workgroup's row sums, added by the first wave's lanes in a fixed butterfly
        static_assert(RPP * R <= 64, "one value per lane");
        __syncthreads();
        if (tid < 64) {
            float t = tid < RPP * R ? sq[tid] : 0.f;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o);
            if (tid == 0) ssq[blockIdx.x] = t;
        }
    }
}

constexpr int kSeqT = 64;         // most time steps per LDS round of the sequential kernel
constexpr int kSeqItems = 4096;   // most x (and B, C) values per round: 16 per thread

__host__ __device__ inline int seq_steps(int Pd, int N) {
    const int w = Pd > N ? Pd : N;
    const int t = kSeqItems / w;
    return t < kSeqT ? (t > 0 ? t : 1) : kSeqT;
}

// Sequential SSD for shapes outside the MFMA kernel (head dim != 64 or d_state not 64/128):
// the one-token update above run over the L steps of a (b, h) sequence with the state in
// registers. Each thread owns RPT rows of the state (RPT <= 8) in float4 columns. The
// steps' inputs come through LDS, kSeqT steps per round, fetched one round ahead.
template <typename TIN, int LPR>
__global__ __launch_bounds__(256) void ssd_seq_kernel(SsdArgs a, int Pd) {
    constexpr int RPP = 256 / LPR;
    constexpr int MAXR = 8;
    constexpr int MAXX = kSeqItems / 256;    // x values per thread and round
    constexpr int MAXBC = kSeqItems / 256;   // B (and C) values per thread and round
    extern __shared__ float seq_smem[];
    const int bh = blockIdx.x;
    const int h = bh % a.H, b = bh / a.H, g = h / (a.H / a.G);
    const int tid = threadIdx.x, c4 = tid % LPR, rsub = tid / LPR;
    const int N = a.N, L = a.L;
    const int T = seq_steps(Pd, N);   // time steps staged per round
    const bool col_ok = 4 * c4 < N;
    const TIN* X = reinterpret_cast<const TIN*>(a.x) + (long)h * Pd;
    const TIN* Bp = reinterpret_cast<const TIN*>(a.Bm) + (long)g * N;
    const TIN* Cp = reinterpret_cast<const TIN*>(a.Cm) + (long)g * N;
    const float Ah = a.A[h], dtb = a.dt_bias ? a.dt_bias[h] : 0.f, Dh = a.Dsk ? a.Dsk[h] : 0.f;
    const long rb = (long)b * L;
    float* xs = seq_smem;                          // [T][Pd]
    float* bs = xs + ((T * Pd + 3) & ~3);          // [T][N], 16-byte aligned for float4 reads
    float* cs = bs + T * N;        // [T][N]
    float* ds = cs + T * N;        // [T]: dt'
    float4 st[MAXR];
#pragma unroll
    for (int k = 0; k < MAXR; ++k) {
        const int p = rsub + k * RPP;
        st[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (a.h0 && p < Pd && col_ok) {
            const float* src = a.h0 + ((long)bh * Pd + p) * N + 4 * c4;
            st[k] = make_float4(src[0], src[1], src[2], src[3]);
        }
    }

    // The inputs of T steps are fetched into registers by the whole workgroup (clamped
    // indices, no branches, so every load is in flight at once), then staged in LDS; the
    // sequential steps read LDS while the next round's loads are in flight.
    float px[MAXX], pb[MAXBC], pc[MAXBC], pdt = 0.f;
    auto fetch = [&](int t0) {
#pragma unroll
        for (int i = 0; i < MAXX; ++i) {
            int e = tid + 256 * i;
            e = e < T * Pd ? e : T * Pd - 1;
            const int t = min(t0 + e / Pd, L - 1);
            px[i] = ld1<TIN>(X + (rb + t) * a.ldx + e % Pd);
        }
#pragma unroll
        for (int i = 0; i < MAXBC; ++i) {
            int e = tid + 256 * i;
            e = e < T * N ? e : T * N - 1;
            const int t = min(t0 + e / N, L - 1);
            pb[i] = ld1<TIN>(Bp + (rb + t) * a.ldb + e % N);
            pc[i] = ld1<TIN>(Cp + (rb + t) * a.ldc + e % N);
        }
        pdt = a.dt[(rb + min(t0 + (tid < T ? tid : 0), L - 1)) * a.lddt + h];
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < MAXX; ++i)
            if (tid + 256 * i < T * Pd) xs[tid + 256 * i] = px[i];
#pragma unroll
        for (int i = 0; i < MAXBC; ++i)
            if (tid + 256 * i < T * N) {
                bs[tid + 256 * i] = pb[i];
                cs[tid + 256 * i] = pc[i];
            }
        if (tid < T) {
            float dl = pdt + dtb;
            if (a.softplus) dl = ssm::softplus(dl);
            ds[tid] = fminf(fmaxf(dl, a.dt_min), a.dt_max);
        }
    };
    if (L > 0) {   // (L = 0 passes h0 through to hT)
        fetch(0);
        stage();
        __syncthreads();
    }
    const int cb = col_ok ? 4 * c4 : 0;
    for (int t0 = 0; t0 < L; t0 += T) {
        fetch(t0 + T < L ? t0 + T : t0);   // the last round refetches its own inputs
        const int tn = min(T, L - t0);
        for (int tt = 0; tt < tn; ++tt) {
            const float dl = ds[tt];
            const float dA = ssm::ex2(dl * Ah * ssm::kLog2e);
            const float4 bq = *reinterpret_cast<const float4*>(bs + tt * N + cb);
            const float4 cq = *reinterpret_cast<const float4*>(cs + tt * N + cb);
            const float bv[4] = {col_ok ? bq.x : 0.f, col_ok ? bq.y : 0.f, col_ok ? bq.z : 0.f,
                                 col_ok ? bq.w : 0.f};
            const float cv[4] = {cq.x, cq.y, cq.z, cq.w};
            const long r = rb + t0 + tt;
#pragma unroll
            for (int k = 0; k < MAXR; ++k) {
                const int p = rsub + k * RPP;
                if (p >= Pd) break;
                const float xp = xs[tt * Pd + p];
                const float dx = dl * xp;
                float4& v = st[k];
                v.x = fmaf(dA, v.x, dx * bv[0]);
                v.y = fmaf(dA, v.y, dx * bv[1]);
                v.z = fmaf(dA, v.z, dx * bv[2]);
                v.w = fmaf(dA, v.w, dx * bv[3]);
                float acc = v.x * cv[0] + v.y * cv[1] + v.z * cv[2] + v.w * cv[3];
#pragma unroll
                for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, LPR);
                if (c4 == 0) a.y[r * a.ldy + (long)h * Pd + p] = fmaf(Dh, xp, acc);
            }
        }
        __syncthreads();
        stage();
        __syncthreads();
    }
    if (a.hT) {
#pragma unroll
        for (int k = 0; k < MAXR; ++k) {
            const int p = rsub + k * RPP;
            if (p < Pd && col_ok) {
                float* dst = a.hT + ((long)bh * Pd + p) * N + 4 * c4;
                dst[0] = st[k].x; dst[1] = st[k].y; dst[2] = st[k].z; dst[3] = st[k].w;
            }
        }
    }
}

template <typename TIN>
ssm_status launch_ssd_seq(SsdArgs& a, int Pd, hipStream_t st) {
    if (a.N % 4 != 0)
        return ssm::fail(SSM_ERR_UNSUPPORTED, "ssd: d_state %d is not a multiple of 4", a.N);
    const int lpr = a.N / 4;
    int L2 = 1;
    while (L2 < lpr) L2 <<= 1;
    if (L2 > 64 || Pd > 8 * (256 / L2))
        return ssm::fail(SSM_ERR_UNSUPPORTED, "ssd: head dim %d with d_state %d is too large", Pd,
                         a.N);
    const unsigned grid = (unsigned)(a.B * a.H);
    const int T = seq_steps(Pd, a.N);
    const size_t smem = sizeof(float) * ((((size_t)T * Pd + 3) & ~(size_t)3) + (size_t)T * (2 * a.N + 1));
    switch (L2) {
        case 1: ssd_seq_kernel<TIN, 1><<<grid, 256, smem, st>>>(a, Pd); break;
        case 2: ssd_seq_kernel<TIN, 2><<<grid, 256, smem, st>>>(a, Pd); break;
        case 4: ssd_seq_kernel<TIN, 4><<<grid, 256, smem, st>>>(a, Pd); break;
        case 8: ssd_seq_kernel<TIN, 8><<<grid, 256, smem, st>>>(a, Pd); break;
        case 16: ssd_seq_kernel<TIN, 16><<<grid, 256, smem, st>>>(a, Pd); break;
        case 32: ssd_seq_kernel<TIN, 32><<<grid, 256, smem, st>>>(a, Pd); break;
        default: ssd_seq_kernel<TIN, 64><<<grid, 256, smem, st>>>(a, Pd); break;
    }
    return ssm::check_launch("ssd_seq");
}

// Shapes outside the MFMA kernel with one group, d_state <= 64 and fp32 inputs run as the
// Mamba-1 chunked scan over D = H*P channels: channel h*P + p has dt[b, t, h], A[h] for every
// state, dt_bias[h] and D[h], and every channel reads the same B and C. This kernel writes
// those per-channel copies to the workspace (dt: (B, L, D); A: (D, N); bias, D: (D)).
__global__ void ssd_expand_kernel(const float* __restrict__ dt, long lddt,
                                  const float* __restrict__ dt_bias, const float* __restrict__ A,
                                  const float* __restrict__ Dsk, int B, int L, int H, int Pd,
                                  int N, float* __restrict__ dte, float* __restrict__ Ae,
                                  float* __restrict__ be, float* __restrict__ De) {
    const long D = (long)H * Pd;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long nt = (long)B * L * D;
    if (i < nt) {
        const long r = i / D;
        const int h = (int)((i % D) / Pd);
        dte[i] = dt[r * lddt + h];
    } else if (i < nt + D * N) {
        const long k = i - nt;
        Ae[k] = A[(k / N) / Pd];
    } else if (i < nt + D * N + D) {
        const long d = i - nt - D * N;
        be[d] = dt_bias ? dt_bias[d / Pd] : 0.f;
        De[d] = Dsk ? Dsk[d / Pd] : 0.f;
    }
}

size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace of the chunked fallback: the copies above, then the scan's own workspace.
size_t chunked_fallback_bytes(int B, int L, int H, int Pd, int N) {
    const size_t D = (size_t)H * Pd;
    return up256(sizeof(float) * (size_t)B * L * D) + up256(sizeof(float) * D * N) +
           2 * up256(sizeof(float) * D) + ssm_selective_scan_workspace(B, L, (int)D, N);
}

bool chunked_fallback_shape(int Pd, int G, int N) {
    return !(Pd == P && (N == 64 || N == 128)) && G == 1 && N <= 64;
}

}  // namespace

extern "C" size_t ssm_ssd_workspace(int B, int L, int H, int Pd, int G, int N) {
    if (B <= 0 || L <= 0 || H <= 0 || Pd <= 0 || N <= 0) return 0;
    if (chunked_fallback_shape(Pd, G, N)) return chunked_fallback_bytes(B, L, H, Pd, N);
    if (Pd != P || (N != 64 && N != 128)) return 0;
    // the larger of the bf16 kernel's and the fp32 kernel's segment states (the size does
    // not depend on the element type the caller will pass)
    int nchunks, nseg, per;
    plan(B, L, H, nchunks, nseg, per);
    const size_t bf = nseg <= 1 ? 0 : sizeof(float) * (size_t)B * H * nseg * ((size_t)Pd * N + 1);
    return std::max(bf, ssm::ssd_f32_workspace(B, L, H, G, Pd, N));
}

namespace ssm {

// Whether the fp32 matrix-core SSD can also apply the gated RMSNorm's element-wise part (one
// norm group; the offsets and alignments of its fp32 path).
bool ssd_gated_ok(int Pd, int G, int N, long ldx, long lddt, long ldb, long ldc, long ldy,
                  long ldz, const void* x, const void* Bm, const void* Cm, const float* y,
                  const float* z, const float* gn) {
    const long lim = (1L << 31) / Q;
    const bool fit = ldx * 4 < lim && ldb * 4 < lim && ldc * 4 < lim && ldy * 4 < lim &&
                     lddt * 4 < lim && ldz * 4 < lim;
    const bool al = (((uintptr_t)x | (uintptr_t)Bm | (uintptr_t)Cm | (uintptr_t)y |
                      (uintptr_t)z | (uintptr_t)gn) & 15) == 0 &&
                    (ldx | ldb | ldc | ldy | ldz) % 4 == 0;
    return G == 1 && ssd_f32_shape(Pd, N) && fit && al;
}

}  // namespace ssm

extern "C" ssm_status ssm_ssd_chunk_scan(int in_dtype, const void* x, long ldx, const float* dt,
                                         long lddt, const float* dt_bias, int softplus,
                                         float dt_min, float dt_max, const float* A,
                                         const void* Bm, long ldb, const void* Cm, long ldc,
                                         const float* Dsk, float* y, long ldy, int B, int L,
                                         int H, int Pd, int G, int N, const float* h0,
                                         float* hT, void* workspace, size_t workspace_bytes,
                                         void* stream) {
    SSM_REQUIRE(x && dt && A && Bm && Cm && y, "ssm_ssd_chunk_scan: null input");
    SSM_REQUIRE(in_dtype == SSM_F32 || in_dtype == SSM_BF16, "ssm_ssd_chunk_scan: bad dtype");
    SSM_REQUIRE(B >= 0 && L >= 0 && H > 0 && G > 0 && H % G == 0 && Pd > 0 && N > 0,
                "ssm_ssd_chunk_scan: bad shape");
    const long ev = in_dtype == SSM_F32 ? 4 : 8;   // vector-load element alignment
    const long esz = in_dtype == SSM_F32 ? 4 : 2;
    // the MFMA kernel addresses one chunk (Q rows) of every tensor with 32-bit byte offsets
    const long lim = (1L << 31) / Q;
    const bool offsets_fit = ldx * esz < lim && ldb * esz < lim && ldc * esz < lim &&
                             ldy * 4 < lim && lddt * 4 < lim;
    const bool mfma_path = Pd == P && (N == 64 || N == 128) && offsets_fit;
    SSM_REQUIRE(ldx >= (long)H * Pd && ldb >= (long)G * N && ldc >= (long)G * N &&
                    ldy >= (long)H * Pd && lddt >= H,
                "ssm_ssd_chunk_scan: row stride below row width");
    if (mfma_path)
        SSM_REQUIRE(ldx % 4 == 0 && ldy % 4 == 0 && ldb % ev == 0 && ldc % ev == 0 &&
                        (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 &&
                        (uintptr_t)Bm % 16 == 0 && (uintptr_t)Cm % 16 == 0,
                    "ssm_ssd_chunk_scan: x/B/C/y rows must be 16-byte aligned");
    if (B == 0) return SSM_OK;
    if (L == 0) {
        if (hT) {
            const size_t bytes = sizeof(float) * (size_t)B * H * Pd * N;
            if (h0) SSM_HIP_TRY(hipMemcpyAsync(hT, h0, bytes, hipMemcpyDeviceToDevice,
                                               (hipStream_t)stream));
            else SSM_HIP_TRY(hipMemsetAsync(hT, 0, bytes, (hipStream_t)stream));
        }
        return SSM_OK;
    }
    SsdArgs a{};
    a.x = x; a.ldx = ldx; a.dt = dt; a.lddt = lddt; a.dt_bias = dt_bias; a.softplus = softplus;
    a.dt_min = dt_min; a.dt_max = dt_max; a.A = A; a.Bm = Bm; a.ldb = ldb; a.Cm = Cm;
    a.ldc = ldc; a.Dsk = Dsk; a.y = y; a.ldy = ldy; a.B = B; a.L = L; a.H = H; a.G = G; a.N = N;
    a.h0 = h0; a.hT = hT;
    hipStream_t st = (hipStream_t)stream;
    // the Mamba-1 scan has no dt clamp: it stands in when the clamp cannot bind
    const bool no_clamp = (softplus && dt_min <= 0.f && dt_max == INFINITY) ||
                          (dt_min == -INFINITY && dt_max == INFINITY);
    if (!mfma_path && in_dtype == SSM_F32 && no_clamp && chunked_fallback_shape(Pd, G, N) &&
        workspace && workspace_bytes >= chunked_fallback_bytes(B, L, H, Pd, N)) {
        const long D = (long)H * Pd;
        char* p = (char*)workspace;
        float* dte = (float*)p;
        p += up256(sizeof(float) * (size_t)B * L * D);
        float* Ae = (float*)p;
        p += up256(sizeof(float) * (size_t)D * N);
        float* be = (float*)p;
        p += up256(sizeof(float) * (size_t)D);
        float* De = (float*)p;
        p += up256(sizeof(float) * (size_t)D);
        const long n = (long)B * L * D + D * N + D;
        ssd_expand_kernel<<<(unsigned)ssm::cdiv(n, 256), 256, 0, st>>>(
            dt, lddt, dt_bias, A, Dsk, B, L, H, Pd, N, dte, Ae, be, De);
        SSM_HIP_TRY(hipGetLastError());
        const size_t rest = workspace_bytes - (size_t)(p - (char*)workspace);
        return ssm_selective_scan((const float*)x, ldx, dte, D, be, softplus, Ae,
                                  (const float*)Bm, ldb, (const float*)Cm, ldc, Dsk ? De : nullptr,
                                  nullptr, 0, y, ldy, B, L, (int)D, N, h0, hT, p, rest, stream);
    }
    if (!mfma_path)
        return in_dtype == SSM_F32 ? launch_ssd_seq<float>(a, Pd, st)
                                   : launch_ssd_seq<__bf16>(a, Pd, st);
    if (in_dtype == SSM_F32)
        return ssm::ssd_f32((const float*)x, ldx, dt, lddt, dt_bias, softplus, dt_min, dt_max, A,
                            (const float*)Bm, ldb, (const float*)Cm, ldc, Dsk, y, ldy, B, L, H, G,
                            N, h0, hT, workspace, workspace_bytes, st);
    plan(B, L, H, a.nchunks, a.nseg, a.chunks_per_seg);
    if (a.nseg > 1) {
        // the bf16 kernel's own part: the segment states and decays
        const size_t need = sizeof(float) * (size_t)B * H * a.nseg * ((size_t)P * N + 1);
        SSM_REQUIRE(workspace && workspace_bytes >= need,
                    "ssm_ssd_chunk_scan: workspace of %zu bytes needed",
                    ssm_ssd_workspace(B, L, H, Pd, G, N));
        a.seg_state = (float*)workspace;
        a.seg_decay = a.seg_state + (size_t)B * H * a.nseg * P * N;
    }
    // two heads per workgroup when head pairs share a group
    if ((H / G) % 2 == 0)
        return N == 128 ? launch_ssd<128, 2>(a, st) : launch_ssd<64, 2>(a, st);
    return N == 128 ? launch_ssd<128, 1>(a, st) : launch_ssd<64, 1>(a, st);
}

extern "C" ssm_status ssm_m2_state_update(const float* x, long ldx, const float* dt, long lddt,
                                          const float* dt_bias, int softplus, float dt_min,
                                          float dt_max, const float* A, const float* Bm,
                                          long ldb, const float* Cm, long ldc, const float* Dsk,
                                          const float* z, long ldz, float* y, long ldy, float* h,
                                          int B, int H, int Pd, int G, int N, void* stream) {
    SSM_REQUIRE(x && dt && A && Bm && Cm && y && h, "ssm_m2_state_update: null input");
    SSM_REQUIRE(B >= 0 && H > 0 && G > 0 && H % G == 0 && Pd > 0, "ssm_m2_state_update: bad shape");
    if (!(N == 8 || N == 16 || N == 32 || N == 64 || N == 128 || N == 256))
        return ssm::fail(SSM_ERR_UNSUPPORTED, "ssm_m2_state_update: d_state %d not in {8..256}", N);
    SSM_REQUIRE(ldb % 4 == 0 && ldc % 4 == 0 && (uintptr_t)Bm % 16 == 0 &&
                    (uintptr_t)Cm % 16 == 0 && (uintptr_t)h % 16 == 0,
                "ssm_m2_state_update: B/C/state must be 16-byte aligned");
    if (B == 0) return SSM_OK;
    hipStream_t st = (hipStream_t)stream;
    const int lpr = N / 4, rpp = 256 / lpr;
    // two rows per thread (R = 2): B*H*ceil(P / (2*rpp)) workgroups
    constexpr int R = 2;
    const int bph = (int)ssm::cdiv(Pd, rpp * R);
    const unsigned grid = (unsigned)((long)B * H * bph);
    const bool full = Pd % (rpp * R) == 0;
#define M2U(LPR)                                                                             \
    (full ? m2_update_kernel<LPR, R, false, true><<<grid, 256, 0, st>>>(                    \
                x, ldx, dt, lddt, dt_bias, softplus, dt_min, dt_max, A, Bm, ldb, Cm, ldc, Dsk, \
                z, ldz, nullptr, nullptr, y, ldy, h, H, Pd, G, N, bph)                       \
          : m2_update_kernel<LPR, R, false, false><<<grid, 256, 0, st>>>(                   \
                x, ldx, dt, lddt, dt_bias, softplus, dt_min, dt_max, A, Bm, ldb, Cm, ldc, Dsk, \
                z, ldz, nullptr, nullptr, y, ldy, h, H, Pd, G, N, bph))
    switch (lpr) {
        case 2: M2U(2); break;
        case 4: M2U(4); break;
        case 8: M2U(8); break;
        case 16: M2U(16); break;
        case 32: M2U(32); break;
        default: M2U(64); break;
    }
#undef M2U
    return ssm::check_launch("m2_state_update");
}

namespace ssm {

// Two state rows per thread, as in ssm_m2_state_update: P / (2 * 256 / (N / 4)) workgroups
// per (b, h), each one partial sum.
int m2_gated_nssq(int H, int P, int N) {
    const int rpp = 256 / (N / 4);
    return H * (int)cdiv(P, rpp * 2);
}

ssm_status launch_m2_update_gated(const float* x, long ldx, const float* dt, long lddt,
                                  const float* dt_bias, const float* A, const float* Bm, long ldb,
                                  const float* Cm, long ldc, const float* Dsk, const float* z,
                                  long ldz, const float* gn, float* y, float* ssq, float* h,
                                  int B, int H, int Pd, int G, int N, hipStream_t st) {
    SSM_REQUIRE(x && dt && A && Bm && Cm && z && gn && y && ssq && h, "m2_update_gated: null");
    SSM_REQUIRE((H * Pd) % 16 == 0, "m2_update_gated: d_inner %d not a multiple of 16", H * Pd);
    SSM_REQUIRE(N == 64 || N == 128 || N == 256, "m2_update_gated: d_state %d", N);
    SSM_REQUIRE(ldb % 4 == 0 && ldc % 4 == 0 && (uintptr_t)Bm % 16 == 0 &&
                    (uintptr_t)Cm % 16 == 0 && (uintptr_t)h % 16 == 0,
                "m2_update_gated: B/C/state must be 16-byte aligned");
    if (B == 0) return SSM_OK;
    constexpr int R = 2;
    const int lpr = N / 4, rpp = 256 / lpr;
    const int bph = (int)cdiv(Pd, rpp * R);
    const unsigned grid = (unsigned)((long)B * H * bph);
    const bool full = Pd % (rpp * R) == 0;
#define M2G(LPR)                                                                            \
    (full ? m2_update_kernel<LPR, R, true, true><<<grid, 256, 0, st>>>(                    \
                x, ldx, dt, lddt, dt_bias, 1, 0.f, INFINITY, A, Bm, ldb, Cm, ldc, Dsk, z,    \
                ldz, gn, ssq, y, 0, h, H, Pd, G, N, bph)                                    \
          : m2_update_kernel<LPR, R, true, false><<<grid, 256, 0, st>>>(                   \
                x, ldx, dt, lddt, dt_bias, 1, 0.f, INFINITY, A, Bm, ldb, Cm, ldc, Dsk, z,    \
                ldz, gn, ssq, y, 0, h, H, Pd, G, N, bph))
    switch (lpr) {
        case 16: M2G(16); break;
        case 32: M2G(32); break;
        default: M2G(64); break;
    }
#undef M2G
    return check_launch("m2_update_gated");
}

}  // namespace ssm
