// K3-K6 for float32 inputs: the Mamba-2 SSD (Dao & Gu 2024, section 6) in full fp32
// arithmetic on the gfx950 fp32 matrix cores (v_mfma_f32_16x16x4_f32), so every product and
// sum is an fp32 operation, as in the fp32 WGSL kernels this backend replaces.
//
// Work split. One workgroup owns one (batch, segment) and HPW heads of one group (two when
// the heads per group are even, else one); four waves per head own the four 16-row blocks of
// the head dim (wave w of a head: p = 16w .. 16w+15) and walk the segment's chunks of
// QF = 32 time steps in order. B, C and the raw C B^T tiles depend on the group only, so a
// two-head workgroup stages B and C once, and the C B^T tiles are formed once per (batch,
// group, chunk) by a pre-pass (ssd_f32_cb_kernel, into the workspace) and prefetched a chunk
// ahead, one tile per wave, then scaled into both heads' M^T; without room for them in the
// workspace the workgroup forms each tile once itself. Between the chunk's two barriers the
// tiles were the MFMA work of three waves while the others waited (the pre-pass took cfg3
// from 693 to 645 µs plus 9.5 µs for the pre-pass, same bits). A small chunk is the cheaper
// one here: the state never leaves the registers,
// so nothing is paid per chunk in memory, while the quadratic in-chunk terms (C B^T and its
// product with X) shrink with the chunk.
//
// Per chunk, with acum_t the running sum of dt' A_h over the chunk (kept in log2 units):
//   M^T[i][j] = (C B^T)[i][j] * 2^(acum_i - acum_j) * dt'_j  (j <= i),  + D_h on j == i
//               the causal 16x16 tiles are shared out over the waves; K = N
//   Y^T[p][i] = 2^acum_i * sum_n S[p][n] C[i][n]             (K = N, entering state)
//             + sum_j X^T[p][j] M^T[i][j]                     (K = j)
//   S^T[n][p] = 2^acum_end S^T[n][p] + sum_j B[j][n] (X[j][p] w_j),  w_j = 2^(acum_end - acum_j) dt'_j
//
// Register layouts. In a 16x16x4 MFMA, lane l supplies A[l % 16][k] and B[k][l % 16] for one
// k (k = l / 16 in the instruction's own numbering) and gets D[4 (l / 16) + r][l % 16] back
// in register r. Here lane group g = l / 16 supplies k = 4g + s of a 16-wide k block in MFMA
// s = 0..3: the four MFMAs cover the block once, and a permutation of k applied to both
// operands leaves the sum unchanged.
// Then:
//   - the state accumulator of S^T tile (n block nb) holds S^T[16nb + 4g + r][16w + l % 16],
//     which is the A operand S[p = 16w + l%16][n = 16nb + 4g + r] of MFMA r for Y_off: the
//     entering state goes from the accumulators into the next product without a copy;
//   - the C B^T accumulator (rows j, columns i) holds M^T[i][j] for four consecutive j, which
//     are written to LDS as one 16-byte row piece and read back as the B operand of Y_diag;
//   - X[j][p] for the lane's j values is loaded from global memory straight into registers;
//     times w_j it is the B operand of the state update.
// B and C rows are staged in LDS (double-buffered, so staging the next chunk needs no barrier
// after the state update); two barriers per chunk: after staging and after M^T.
//
// Long single sequences with few heads are cut into segments as in the bf16 kernel: a
// state-only pass gives each segment's local final state and total decay, a combine pass
// turns them into entering states, and the full pass starts every segment from its own.
#include <algorithm>

#include "common.hpp"
#include "ssd.hpp"

namespace {

constexpr int QF = 32;       // time steps per chunk
constexpr int PF = 64;       // head dim
constexpr int kTargetWG = 512;

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct F32Args {
    const float* x; long ldx;
    const float* dt; long lddt;
    const float* dt_bias; int softplus; float dt_min, dt_max;
    const float* A;
    const float* Bm; long ldb;
    const float* Cm; long ldc;
    const float* Dsk;
    float* y; long ldy;
    int B, L, H, G;
    int nchunks, nseg, chunks_per_seg;
    const float* h0;
    float* hT;
    float* seg_state;   // (B,H,nseg,P,N)
    float* seg_decay;   // (B,H,nseg)
    // given: the raw C B^T tiles of every (batch, group, chunk) from ssd_f32_cb_kernel,
    // (B, G, nchunks, 3 tiles, 64 lanes, 4) in accumulator order; else the full pass forms them
    const float* cbw;
    int remap;
    // gated output (GATED): y <- u * gn with u = y * silu(z), and ssq (B*L, H) = sum over the
    // head's P channels of u^2 (the gated RMSNorm's element-wise part and its partial sums)
    const float* z; long ldz;
    const float* gn;
    float* ssq;
};

template <int NN, bool FULL, bool GATED, int HPW>
struct SmemF32 {
    static constexpr int BP = NN + 4;    // B / C row pitch (floats): b128 rows conflict-free
    static constexpr int MP = QF + 4;    // M^T row pitch
    float b[2][QF][BP];                                  // B (j, n), two chunks
    float c[FULL ? 2 : 1][FULL ? QF : 1][BP];            // C (i, n), two chunks
    float m[HPW][FULL ? QF : 1][MP];                     // M^T (i, j) per head
    float ac[2][HPW][QF];    // acum_t in log2 units
    float dv[2][HPW][QF];    // dt'_t
    float wj[2][HPW][QF];    // w_t = 2^(acum_end - acum_t) dt'_t
    float ae[2][HPW];        // acum_end
    float sq[GATED ? 2 : 1][HPW][GATED ? 4 : 1][GATED ? QF : 1];   // per-wave sums of u^2 per row
};

using ssm::bload16;
using ssm::bload4;
using ssm::bstore16;
using ssm::rsrc;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float add_dpp(float x) {
    const int y = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xf,
                                              true);
    return x + __builtin_bit_cast(float, y);
}

// Inclusive prefix sum over the 64 lanes (row_shr within rows of 16, then row_bcast).
__device__ __forceinline__ float wave_prefix_sum(float v) {
    v = add_dpp<0x111, 0xf>(v);
    v = add_dpp<0x112, 0xf>(v);
    v = add_dpp<0x114, 0xf>(v);
    v = add_dpp<0x118, 0xf>(v);
    v = add_dpp<0x142, 0xa>(v);
    v = add_dpp<0x143, 0xc>(v);
    return v;
}

__device__ __forceinline__ float4 as_f4(floatx4 v) { return make_float4(v[0], v[1], v[2], v[3]); }

template <int NN, bool FULL, bool GATED = false, int HPW = 1>
__global__ __launch_bounds__(256 * HPW, 2) void ssd_f32_kernel(F32Args a) {
    static_assert(FULL || HPW == 1, "the state-only pass takes one head per workgroup");
    __shared__ __attribute__((aligned(16))) SmemF32<NN, FULL, GATED, HPW> sm;
    using SM = SmemF32<NN, FULL, GATED, HPW>;
    constexpr int NB = NN / 16;          // n blocks (state tiles per wave, k groups of C B^T)
    constexpr int QB = QF / 16;          // time blocks per chunk
    constexpr int NCB = QB * (QB + 1) / 2;   // causal C B^T tiles per chunk
    static_assert(NCB == 3, "three tiles over four waves: one wave per chunk has no tile");
    constexpr int RL = NN / 4;           // lanes per staged B / C row (one float4 each)
    constexpr int RPP = 256 * HPW / RL;  // rows per staging pass
    constexpr int SP = QF / RPP;         // staging passes

    int wg = blockIdx.x;
    if (a.remap) {
        const int per = gridDim.x / 8;
        wg = (blockIdx.x % 8) * per + blockIdx.x / 8;
    }
    // segment-major: the heads of one (batch, segment) are adjacent and, after the remap, on
    // one XCD, where they share that segment's B and C rows through L2. With HPW = 2 the
    // workgroup takes heads 2k and 2k + 1 of one group: wave w works on head w / 4 of the
    // workgroup (its state rows p = 16 (w % 4) .. + 15), and B, C and the C B^T tiles serve
    // both heads.
    const int HW = a.H / HPW;
    const int seg = wg / (a.B * HW);
    const int bhw = wg % (a.B * HW);
    const int b = bhw / HW;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hw = w >> 2, wl = w & 3;
    const int h0w = HPW * (bhw % HW);    // the workgroup's first head
    const int h = h0w + hw;
    const int bh = b * a.H + h;
    const int g = h / (a.H / a.G);
    const int l16 = lane & 15, q4 = lane >> 4;
    const int p0 = 16 * wl;
    const int sr = tid / RL, sc4 = 4 * (tid % RL);   // staging row / column

    const float Ah = a.A[h] * ssm::kLog2e;
    const float dtb = a.dt_bias ? a.dt_bias[h] : 0.f;
    float Dh[HPW];   // D of the workgroup's heads (the C B^T tiles serve them all)
#pragma unroll
    for (int k = 0; k < HPW; ++k) Dh[k] = a.Dsk ? a.Dsk[h0w + k] : 0.f;
    // gated output: this lane's four norm weights (columns p0 + 4 q4 .. + 3 of the head)
    float4 gw = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (GATED) gw = *reinterpret_cast<const float4*>(a.gn + (long)h * PF + p0 + 4 * q4);

    const int c_begin = seg * a.chunks_per_seg;
    const int c_end = min(c_begin + a.chunks_per_seg, a.nchunks);

    const long brow = (long)b * a.L;
    const float* x0 = a.x + brow * a.ldx + (long)h * PF + p0;   // wave-uniform base
    const float* b0 = a.Bm + brow * a.ldb + (long)g * NN;
    const float* cm0 = a.Cm + brow * a.ldc + (long)g * NN;
    const float* d0 = a.dt + brow * a.lddt + h;
    auto rows_of = [&](int c) { return c < c_end ? min(QF, a.L - c * QF) : 0; };
    // ssq[(b L + t) H + h] for row t of chunk c and head h0w + tid / QF from the head's four
    // waves' partial sums (threads tid < HPW QF)
    auto flush_ssq = [&](int c, int bf) {
        const int hk = tid / QF, tt = tid % QF;
        const int t = c * QF + tt;
        if (t < a.L) {
            const float v = (sm.sq[bf][hk][0][tt] + sm.sq[bf][hk][1][tt]) +
                            (sm.sq[bf][hk][2][tt] + sm.sq[bf][hk][3][tt]);
            a.ssq[(brow + t) * a.H + h0w + hk] = v;
        }
    };
    auto span = [](int qv, long ld, int width) {
        return qv > 0 ? (unsigned)(((long)(qv - 1) * ld + width) * 4) : 0u;
    };

    // C B^T tiles rotate over the waves from one workgroup to the next, so that no SIMD always
    // gets the wave with the most (or no) tiles; the wave without a tile scans the next chunk.
    // With two heads the first head's waves form the tiles (for both heads) and wave
    // scan_wave of each head scans that head's next chunk.
    const int rot = blockIdx.x & 3;
    const int scan_wave = (NCB + rot) & 3;
    // With a.cbw the tiles come from the pre-pass: this wave's tile (t with (t + rot) & 3 ==
    // wl, on the first head's waves) of chunk c is loaded one chunk ahead into cbv (chunks
    // past the last read zeros).
    const int tw = (wl - rot + 4) & 3;
    const bool cb_wave = FULL && hw == 0 && tw < NCB && a.cbw != nullptr;
    const auto rcb = rsrc(a.cbw ? a.cbw + ((long)b * a.G + g) * a.nchunks * NCB * 256 : a.x,
                          a.cbw ? (unsigned)(a.nchunks * NCB * 256 * 4) : 0u);
    floatx4 cbv{0.f, 0.f, 0.f, 0.f};
    auto load_cb = [&](int c) {
        if (cb_wave) cbv = bload16<floatx4>(rcb, (unsigned)((c * NCB + tw) * 256 + 4 * lane) * 4u);
    };

    // raw inputs of one chunk: X[j = 16 jb + 4 q4 + s][p0 + l16], B and C staging rows, dt
    struct Raw {
        float x[QB][4];
        float4 b[SP];
        float4 c[FULL ? SP : 1];
        float4 z[GATED ? QB : 1];   // gated output: z of the lane's y pieces
        float dt;
    } raw;
    // x, B, C (and z) of chunk c and dt of chunk cd (the full pass reads dt one chunk further
    // ahead: its scan runs a chunk early, below)
    auto load_raw = [&](int c, int cd) {
        const int qv = rows_of(c);
        const long r0 = (long)c * QF;
        // dt: one strided 4-byte value per step (a cache line per lane); in the full pass only
        // the wave that scans fetches it, the others get an empty descriptor (no traffic)
        const auto rd = rsrc(d0 + (long)cd * QF * a.lddt,
                             (FULL && wl != scan_wave) ? 0u : span(rows_of(cd), a.lddt, 1));
        const auto rx = rsrc(x0 + r0 * a.ldx, span(qv, a.ldx, 16));
        const auto rb = rsrc(b0 + r0 * a.ldb, span(qv, a.ldb, NN));
        raw.dt = bload4(rd, (unsigned)(lane * a.lddt) * 4u);
#pragma unroll
        for (int jb = 0; jb < QB; ++jb)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                raw.x[jb][s] = bload4(rx, (unsigned)((16 * jb + 4 * q4 + s) * a.ldx + l16) * 4u);
#pragma unroll
        for (int k = 0; k < SP; ++k)
            raw.b[k] = bload16<float4>(rb, (unsigned)((sr + RPP * k) * a.ldb + sc4) * 4u);
        if constexpr (FULL) {
            const auto rc = rsrc(cm0 + r0 * a.ldc, span(qv, a.ldc, NN));
#pragma unroll
            for (int k = 0; k < SP; ++k)
                raw.c[k] = bload16<float4>(rc, (unsigned)((sr + RPP * k) * a.ldc + sc4) * 4u);
        }
        if constexpr (GATED) {
            // issued last: the chunk's first wait (for B and C) does not wait for them
            const auto rz = rsrc(a.z + (brow + r0) * a.ldz + (long)h * PF, span(qv, a.ldz, PF));
#pragma unroll
            for (int ib = 0; ib < QB; ++ib)
                raw.z[ib] = bload16<float4>(rz, (unsigned)((16 * ib + l16) * a.ldz + p0 + 4 * q4) * 4u);
        }
    };

    // entering state: S^T tile nb holds S[p0 + l16][16 nb + 4 q4 + r] in register r
    const float* init = nullptr;
    if (FULL) {
        if (a.nseg > 1) init = a.seg_state + ((long)bh * a.nseg + seg) * PF * NN;
        else if (a.h0) init = a.h0 + (long)bh * PF * NN;
    }
    floatx4 S[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        if (init) {
            const float4 v = *reinterpret_cast<const float4*>(init + (long)(p0 + l16) * NN + 16 * nb + 4 * q4);
            S[nb] = floatx4{v.x, v.y, v.z, v.w};
        } else {
            S[nb] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
    bool state_live = init != nullptr;
    float decay_sum = 0.f;
    // dt' of chunk cc (0 past the segment), its running sum times A_h and the weights w_t into
    // LDS buffer bf (lane = time step)
    auto scan_put = [&](int cc, float raw_dt, int bf) {
        const int qv = rows_of(cc);
        float dv = raw_dt + dtb;
        if (a.softplus) dv = ssm::softplus_fast(dv);
        dv = lane < qv ? fminf(fmaxf(dv, a.dt_min), a.dt_max) : 0.f;
        const float sc = wave_prefix_sum(dv * Ah);
        const float ae = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), QF - 1));
        if (lane < QF) {
            sm.ac[bf][hw][lane] = sc;
            sm.dv[bf][hw][lane] = dv;
            sm.wj[bf][hw][lane] = ssm::ex2(ae - sc) * dv;
        }
        if (lane == 0) sm.ae[bf][hw] = ae;
    };

    if constexpr (FULL) {
        // the first chunk's scan (the loop's wave without a C B^T tile scans the next chunk
        // while the others form their tiles); dt of the second chunk comes with the inputs
        const int qv0 = rows_of(c_begin);
        const auto rd0 = rsrc(d0 + (long)c_begin * QF * a.lddt, span(qv0, a.lddt, 1));
        if (wl == 0) scan_put(c_begin, bload4(rd0, (unsigned)(lane * a.lddt) * 4u), c_begin & 1);
        load_cb(c_begin);
        load_raw(c_begin, c_begin + 1);
    } else {
        load_raw(c_begin, c_begin);
    }
    if constexpr (FULL) {
        // Stores into an empty range (dropped by the range check) make the memory operations
        // in flight at loop entry match the back edge (the prefetch, then the chunk's y
        // stores), so that the wait for the prefetched dt and X never waits for y stores.
        const auto none = rsrc(a.y, 0u);
#pragma unroll
        for (int ib = 0; ib < QB; ++ib) bstore16(make_float4(0.f, 0.f, 0.f, 0.f), none, 16u * ib);
    }
    for (int c = c_begin; c < c_end; ++c) {
        const int buf = c & 1;
        const int qv = min(QF, a.L - c * QF);
        const long row0 = brow + (long)c * QF;

        // ---- dt' and its running sum times A_h (state-only pass: every wave, lane = time
        // step; the full pass formed them a chunk earlier)
        float acend = 0.f;
        if constexpr (!FULL) {
            float dv = raw.dt + dtb;
            if (a.softplus) dv = ssm::softplus_fast(dv);
            dv = lane < qv ? fminf(fmaxf(dv, a.dt_min), a.dt_max) : 0.f;
            const float sc = wave_prefix_sum(dv * Ah);
            acend = __builtin_bit_cast(
                float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), QF - 1));
            decay_sum += acend;
            if (w == 0 && lane < QF) {
                sm.ac[buf][0][lane] = sc;
                sm.dv[buf][0][lane] = dv;
                sm.wj[buf][0][lane] = ssm::ex2(acend - sc) * dv;
            }
        }
        // ---- stage B (and C) rows
#pragma unroll
        for (int k = 0; k < SP; ++k) {
            *reinterpret_cast<float4*>(&sm.b[buf][sr + RPP * k][sc4]) = raw.b[k];
            if constexpr (FULL) *reinterpret_cast<float4*>(&sm.c[buf][sr + RPP * k][sc4]) = raw.c[k];
        }
        float xv[QB][4];
#pragma unroll
        for (int jb = 0; jb < QB; ++jb)
#pragma unroll
            for (int s = 0; s < 4; ++s) xv[jb][s] = raw.x[jb][s];
        __syncthreads();
        // past the segment: an empty range, the loads return zeros. The full pass issues the
        // next chunk's loads after its second barrier, so that the C B^T tiles start at once.
        const float dnext = raw.dt;   // full pass: dt of chunk c + 1
        if constexpr (!FULL) load_raw(c + 1, c + 1);
        if constexpr (GATED) {
            // the previous chunk's row sums of u^2, added over the four waves in order
            if (c > c_begin && tid < HPW * QF) flush_ssq(c - 1, buf ^ 1);
        }

        if constexpr (FULL) {
            // ---- M^T tiles of C B^T (this wave's share of the causal tiles)
            // the wave without a tile scans chunk c + 1 into the other buffers (the last reads
            // of those, chunk c - 1's, came before barrier 1)
            if (wl == scan_wave) scan_put(c + 1, dnext, buf ^ 1);
#pragma unroll
            for (int t = 0; t < NCB; ++t) {
                if (hw != 0 || ((t + rot) & 3) != wl) continue;
                // tile t -> (ib, jb) with jb <= ib, row-major over the lower triangle
                int ib = 0, jb = t;
                while (jb > ib) { jb -= ib + 1; ++ib; }
                // k = n in blocks of 16 (kk); kk and kk + 1 go to two accumulators whose MFMAs
                // alternate, and the next pair's operands are read while this pair multiplies
                floatx4 acc0{0.f, 0.f, 0.f, 0.f}, acc1{0.f, 0.f, 0.f, 0.f};
                if (!cb_wave) {
                const float* brw = &sm.b[buf][16 * jb + l16][4 * q4];
                const float* crw = &sm.c[buf][16 * ib + l16][4 * q4];
                float4 opv[2][4];
                auto ld_pair = [&](int kk, float4* o) {
                    o[0] = *reinterpret_cast<const float4*>(brw + 16 * kk);
                    o[1] = *reinterpret_cast<const float4*>(crw + 16 * kk);
                    o[2] = *reinterpret_cast<const float4*>(brw + 16 * kk + 16);
                    o[3] = *reinterpret_cast<const float4*>(crw + 16 * kk + 16);
                };
                ld_pair(0, opv[0]);
#pragma unroll
                for (int kp = 0; kp < NB / 2; ++kp) {
                    if (kp + 1 < NB / 2) ld_pair(2 * kp + 2, opv[(kp + 1) & 1]);
                    __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the MFMAs
                    const float4* o = opv[kp & 1];
                    acc0 = mfma4(o[0].x, o[1].x, acc0);
                    acc1 = mfma4(o[2].x, o[3].x, acc1);
                    acc0 = mfma4(o[0].y, o[1].y, acc0);
                    acc1 = mfma4(o[2].y, o[3].y, acc1);
                    acc0 = mfma4(o[0].z, o[1].z, acc0);
                    acc1 = mfma4(o[2].z, o[3].z, acc1);
                    acc0 = mfma4(o[0].w, o[1].w, acc0);
                    acc1 = mfma4(o[2].w, o[3].w, acc1);
                }
                }
                // acc0[r] + acc1[r] = (C B^T)[i = 16 ib + l16][j = 16 jb + 4 q4 + r] (from the
                // pre-pass: cbv[r], the same sum); M^T of each head
                const int i = 16 * ib + l16;
#pragma unroll
                for (int k = 0; k < HPW; ++k) {
                    const float aci = sm.ac[buf][k][i];
                    const float4 acj = *reinterpret_cast<const float4*>(&sm.ac[buf][k][16 * jb + 4 * q4]);
                    const float4 dvj = *reinterpret_cast<const float4*>(&sm.dv[buf][k][16 * jb + 4 * q4]);
                    const float acja[4] = {acj.x, acj.y, acj.z, acj.w};
                    const float dvja[4] = {dvj.x, dvj.y, dvj.z, dvj.w};
                    float mv[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int j = 16 * jb + 4 * q4 + r;
                        // the masked (j > i) exponent may overflow: select, never multiply by 0
                        const float cbs = cb_wave ? cbv[r] : acc0[r] + acc1[r];
                        const float f = cbs * (ssm::ex2(aci - acja[r]) * dvja[r]);
                        mv[r] = j < i ? f : (j == i ? f + Dh[k] : 0.f);
                    }
                    *reinterpret_cast<float4*>(&sm.m[k][i][16 * jb + 4 * q4]) =
                        make_float4(mv[0], mv[1], mv[2], mv[3]);
                }
            }
            __syncthreads();   // M^T visible
            // this chunk's z leaves the prefetch registers before the next chunk's loads
            float4 zc[GATED ? QB : 1];
#pragma unroll
            for (int ib = 0; ib < (GATED ? QB : 1); ++ib) zc[ib] = raw.z[ib];
            load_cb(c + 1);
            load_raw(c + 1, c + 2);

            // ---- Y^T[p][i] for the wave's 16 p and the chunk's QF rows i
            floatx4 Y[QB];
#pragma unroll
            for (int ib = 0; ib < QB; ++ib) Y[ib] = floatx4{0.f, 0.f, 0.f, 0.f};
            if (state_live) {
                // C pieces of the next n block are read while this block multiplies; the
                // MFMAs alternate between the row blocks' accumulators
                float4 cq[2][QB];
                auto ld_c = [&](int nb, float4* o) {
#pragma unroll
                    for (int ib = 0; ib < QB; ++ib)
                        o[ib] = *reinterpret_cast<const float4*>(&sm.c[buf][16 * ib + l16][16 * nb + 4 * q4]);
                };
                ld_c(0, cq[0]);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    if (nb + 1 < NB) ld_c(nb + 1, cq[(nb + 1) & 1]);
                    __builtin_amdgcn_sched_barrier(0);
                    const float4* o = cq[nb & 1];
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int ib = 0; ib < QB; ++ib) {
                            const float cvr = r == 0 ? o[ib].x : r == 1 ? o[ib].y : r == 2 ? o[ib].z : o[ib].w;
                            Y[ib] = mfma4(S[nb][r], cvr, Y[ib]);
                        }
                }
#pragma unroll
                for (int ib = 0; ib < QB; ++ib) Y[ib] *= ssm::ex2(sm.ac[buf][hw][16 * ib + l16]);
            }
#pragma unroll
            for (int ib = 0; ib < QB; ++ib)
#pragma unroll
                for (int jb = 0; jb <= ib; ++jb) {
                    const float4 mv = *reinterpret_cast<const float4*>(&sm.m[hw][16 * ib + l16][16 * jb + 4 * q4]);
                    Y[ib] = mfma4(xv[jb][0], mv.x, Y[ib]);
                    Y[ib] = mfma4(xv[jb][1], mv.y, Y[ib]);
                    Y[ib] = mfma4(xv[jb][2], mv.z, Y[ib]);
                    Y[ib] = mfma4(xv[jb][3], mv.w, Y[ib]);
                }
            // ---- y rows 16 ib + l16, columns p0 + 4 q4 .. +3 (rows past L are dropped)
            const auto ry = rsrc(a.y + row0 * a.ldy + (long)h * PF, span(qv, a.ldy, PF));
            if constexpr (GATED) {
                // u = y silu(z) and u * gn; the row's sum of u^2 over this wave's 16 columns
                // (lane groups q4 added pairwise with xor shuffles: the same bits in each)
#pragma unroll
                for (int ib = 0; ib < QB; ++ib) {
                    const float4 zv = zc[ib];
                    const float u0 = Y[ib][0] * ssm::silu(zv.x), u1 = Y[ib][1] * ssm::silu(zv.y);
                    const float u2 = Y[ib][2] * ssm::silu(zv.z), u3 = Y[ib][3] * ssm::silu(zv.w);
                    float ss = (u0 * u0 + u1 * u1) + (u2 * u2 + u3 * u3);
                    ss += __shfl_xor(ss, 16);
                    ss += __shfl_xor(ss, 32);
                    if (q4 == 0) sm.sq[buf][hw][wl][16 * ib + l16] = ss;
                    bstore16(make_float4(u0 * gw.x, u1 * gw.y, u2 * gw.z, u3 * gw.w), ry,
                             (unsigned)((16 * ib + l16) * a.ldy + p0 + 4 * q4) * 4u);
                }
            } else {
#pragma unroll
                for (int ib = 0; ib < QB; ++ib)
                    bstore16(as_f4(Y[ib]), ry, (unsigned)((16 * ib + l16) * a.ldy + p0 + 4 * q4) * 4u);
            }
        }

        // ---- state: S^T = 2^acum_end S^T + sum_j B[j][n] (X[j][p] w_j)
        {
            if constexpr (FULL) acend = sm.ae[buf][hw];
            const float e = ssm::ex2(acend);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) S[nb] *= e;
            // step k = 4 jb + s takes time step j = 16 jb + 4 q4 + s of this lane group; the B
            // values of step k + 1 are read while step k's NB MFMAs (independent
            // accumulators) run
            float xw[QB][4];
#pragma unroll
            for (int jb = 0; jb < QB; ++jb) {
                const float4 wv = *reinterpret_cast<const float4*>(&sm.wj[buf][hw][16 * jb + 4 * q4]);
                xw[jb][0] = xv[jb][0] * wv.x;
                xw[jb][1] = xv[jb][1] * wv.y;
                xw[jb][2] = xv[jb][2] * wv.z;
                xw[jb][3] = xv[jb][3] * wv.w;
            }
            float bq[2][NB];
            auto ld_b = [&](int k, float* o) {
                const float* row = &sm.b[buf][16 * (k >> 2) + 4 * q4 + (k & 3)][l16];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) o[nb] = row[16 * nb];
            };
            ld_b(0, bq[0]);
#pragma unroll
            for (int k = 0; k < 4 * QB; ++k) {
                if (k + 1 < 4 * QB) ld_b(k + 1, bq[(k + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) S[nb] = mfma4(bq[k & 1][nb], xw[k >> 2][k & 3], S[nb]);
            }
        }
        state_live = true;
    }

    if constexpr (GATED) {
        __syncthreads();
        if (c_end > c_begin && tid < HPW * QF) flush_ssq(c_end - 1, (c_end - 1) & 1);
    }

    // ---- outputs of the state
    float* out = nullptr;
    if (FULL) {
        if (a.hT && seg == a.nseg - 1) out = a.hT + (long)bh * PF * NN;
    } else {
        out = a.seg_state + ((long)bh * a.nseg + seg) * PF * NN;
        if (w == 0 && lane == 0) a.seg_decay[(long)bh * a.nseg + seg] = decay_sum;
    }
    if (out) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            *reinterpret_cast<float4*>(out + (long)(p0 + l16) * NN + 16 * nb + 4 * q4) = as_f4(S[nb]);
    }
}

// Segment entering states: slot[s] <- carry; carry = 2^decay[s] carry + local[s] (decay in
// log2 units).
__global__ void ssd_f32_seg_prefix(F32Args a, int PN) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)a.B * a.H * PN) return;
    ssm::seg_prefix_elem(a.seg_state, a.seg_decay, a.h0, a.nseg, PN, i / PN, (int)(i % PN), 1.f);
}

// The raw C B^T tiles of every chunk, formed once per (batch, group, chunk) for all of the
// group's heads (the full pass would form them once per workgroup of two heads). Wave t of a
// workgroup forms causal tile t with the full pass's own MFMA sequence on the same operand
// values (B and C rows of the chunk, zeros past L), so the tile holds the same bits, and
// stores it in accumulator order, one float4 per lane.
template <int NN>
__global__ __launch_bounds__(192) void ssd_f32_cb_kernel(F32Args a) {
    constexpr int NB = NN / 16;
    constexpr int NCB = 3;
    const int lane = threadIdx.x & 63, t = threadIdx.x >> 6;
    const int l16 = lane & 15, q4 = lane >> 4;
    const long id = blockIdx.x;   // (b, g, c), c fastest
    const int c = (int)(id % a.nchunks);
    const int bg = (int)(id / a.nchunks), g = bg % a.G, b = bg / a.G;
    int ib = 0, jb = t;
    while (jb > ib) { jb -= ib + 1; ++ib; }
    const int qv = min(QF, a.L - c * QF);
    const long r0 = (long)b * a.L + (long)c * QF;
    const auto rb = rsrc(a.Bm + r0 * a.ldb + (long)g * NN, (unsigned)(((long)(qv - 1) * a.ldb + NN) * 4));
    const auto rc = rsrc(a.Cm + r0 * a.ldc + (long)g * NN, (unsigned)(((long)(qv - 1) * a.ldc + NN) * 4));
    float4 bo[NB], co[NB];
#pragma unroll
    for (int kk = 0; kk < NB; ++kk) {
        bo[kk] = bload16<float4>(rb, (unsigned)((16 * jb + l16) * a.ldb + 16 * kk + 4 * q4) * 4u);
        co[kk] = bload16<float4>(rc, (unsigned)((16 * ib + l16) * a.ldc + 16 * kk + 4 * q4) * 4u);
    }
    floatx4 acc0{0.f, 0.f, 0.f, 0.f}, acc1{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kp = 0; kp < NB / 2; ++kp) {
        const float4 o0 = bo[2 * kp], o1 = co[2 * kp], o2 = bo[2 * kp + 1], o3 = co[2 * kp + 1];
        acc0 = mfma4(o0.x, o1.x, acc0);
        acc1 = mfma4(o2.x, o3.x, acc1);
        acc0 = mfma4(o0.y, o1.y, acc0);
        acc1 = mfma4(o2.y, o3.y, acc1);
        acc0 = mfma4(o0.z, o1.z, acc0);
        acc1 = mfma4(o2.z, o3.z, acc1);
        acc0 = mfma4(o0.w, o1.w, acc0);
        acc1 = mfma4(o2.w, o3.w, acc1);
    }
    const floatx4 sum = acc0 + acc1;
    *reinterpret_cast<floatx4*>(const_cast<float*>(a.cbw) + (id * NCB + t) * 256 + 4 * lane) = sum;
}

void plan_f32(int B, int L, int H, int& nchunks, int& nseg, int& per) {
    nchunks = (int)ssm::cdiv(L, QF);
    const long bh = (long)B * H;
    long s = ssm::cdiv(kTargetWG, bh > 0 ? bh : 1);
    if (s > nchunks) s = nchunks;
    if (s < 1) s = 1;
    per = (int)ssm::cdiv(nchunks, s);
    nseg = (int)ssm::cdiv(nchunks, per);
}

template <int NN>
ssm_status launch(F32Args& a, hipStream_t st) {
    if (a.nseg > 1) {
        F32Args s1 = a;
        const int nwg1 = a.B * a.H * (a.nseg - 1);   // the last segment's local state is unused
        s1.remap = (nwg1 % 8 == 0) ? 1 : 0;
        ssd_f32_kernel<NN, false><<<nwg1, 256, 0, st>>>(s1);
        ssm_status e = ssm::check_launch("ssd_f32_state_pass");
        if (e != SSM_OK) return e;
        const long n = (long)a.B * a.H * PF * NN;
        ssd_f32_seg_prefix<<<(unsigned)ssm::cdiv(n, 256), 256, 0, st>>>(a, PF * NN);
        e = ssm::check_launch("ssd_f32_seg_prefix");
        if (e != SSM_OK) return e;
    }
    if (a.cbw) {
        ssd_f32_cb_kernel<NN><<<(unsigned)((long)a.B * a.G * a.nchunks), 192, 0, st>>>(a);
        ssm_status e = ssm::check_launch("ssd_f32_cb");
        if (e != SSM_OK) return e;
    }
    // two heads per workgroup when heads 2k and 2k + 1 share a group
    const int hpw = ((a.H / a.G) % 2 == 0) ? 2 : 1;
    const int nwg = a.B * (a.H / hpw) * a.nseg;
    a.remap = (nwg % 8 == 0) ? 1 : 0;
    if (hpw == 2) {
        if (a.ssq) ssd_f32_kernel<NN, true, true, 2><<<nwg, 512, 0, st>>>(a);
        else ssd_f32_kernel<NN, true, false, 2><<<nwg, 512, 0, st>>>(a);
    } else {
        if (a.ssq) ssd_f32_kernel<NN, true, true><<<nwg, 256, 0, st>>>(a);
        else ssd_f32_kernel<NN, true><<<nwg, 256, 0, st>>>(a);
    }
    return ssm::check_launch("ssd_f32_chunk_scan");
}

}  // namespace

namespace ssm {

bool ssd_f32_shape(int Pd, int N) { return Pd == PF && (N == 64 || N == 128); }

// Workspace: the segment states and decays when the sequence is cut into segments, then
// (at a 256-byte boundary) the C B^T tiles of the pre-pass, 3 KB per (batch, group, chunk).
// A workspace without room for the tiles runs the full pass with its own tiles.
static size_t f32_seg_bytes(int B, int H, int nseg, int Pd, int N) {
    return nseg <= 1 ? 0 : sizeof(float) * (size_t)B * H * nseg * ((size_t)Pd * N + 1);
}
static size_t f32_cb_off(size_t seg) { return (seg + 255) & ~(size_t)255; }
static size_t f32_cb_bytes(int B, int G, int nchunks) {
    return sizeof(float) * (size_t)B * G * nchunks * 3 * 256;
}

size_t ssd_f32_workspace(int B, int L, int H, int G, int Pd, int N) {
    if (!ssd_f32_shape(Pd, N) || B <= 0 || L <= 0 || H <= 0 || G <= 0) return 0;
    int nchunks, nseg, per;
    plan_f32(B, L, H, nchunks, nseg, per);
    return f32_cb_off(f32_seg_bytes(B, H, nseg, Pd, N)) + f32_cb_bytes(B, G, nchunks);
}

ssm_status ssd_f32(const float* x, long ldx, const float* dt, long lddt, const float* dt_bias,
                   int softplus, float dt_min, float dt_max, const float* A, const float* Bm,
                   long ldb, const float* Cm, long ldc, const float* Dsk, float* y, long ldy,
                   int B, int L, int H, int G, int N, const float* h0, float* hT,
                   void* workspace, size_t workspace_bytes, hipStream_t st, const float* z,
                   long ldz, const float* gn, float* ssq) {
    F32Args a{};
    a.z = z; a.ldz = ldz; a.gn = gn; a.ssq = ssq;
    if (ssq) {
        SSM_REQUIRE(z && gn && ldz >= (long)H * PF, "ssd_f32: the gated output needs z and gn");
        SSM_REQUIRE(((uintptr_t)z | (uintptr_t)gn | (uintptr_t)y) % 16 == 0 && ldz % 4 == 0 &&
                        ldy % 4 == 0,
                    "ssd_f32: gated output needs 16-byte aligned z, gn, y rows");
    }
    a.x = x; a.ldx = ldx; a.dt = dt; a.lddt = lddt; a.dt_bias = dt_bias; a.softplus = softplus;
    a.dt_min = dt_min; a.dt_max = dt_max; a.A = A; a.Bm = Bm; a.ldb = ldb; a.Cm = Cm;
    a.ldc = ldc; a.Dsk = Dsk; a.y = y; a.ldy = ldy; a.B = B; a.L = L; a.H = H; a.G = G;
    a.h0 = h0; a.hT = hT;
    plan_f32(B, L, H, a.nchunks, a.nseg, a.chunks_per_seg);
    const size_t seg = f32_seg_bytes(B, H, a.nseg, PF, N);
    if (a.nseg > 1) {
        SSM_REQUIRE(workspace && workspace_bytes >= seg,
                    "ssm_ssd_chunk_scan: workspace of %zu bytes needed",
                    ssd_f32_workspace(B, L, H, G, PF, N));
        a.seg_state = (float*)workspace;
        a.seg_decay = a.seg_state + (size_t)B * H * a.nseg * PF * N;
    }
    const size_t cbo = f32_cb_off(seg);
    if (workspace && ((uintptr_t)workspace & 15) == 0 &&
        workspace_bytes >= cbo + f32_cb_bytes(B, G, a.nchunks))
        a.cbw = (const float*)((char*)workspace + cbo);
    return N == 128 ? launch<128>(a, st) : launch<64>(a, st);
}

}  // namespace ssm
