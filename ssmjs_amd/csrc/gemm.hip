// Prefill projections on the fp32 matrix cores: Y = beta * Y + X W^T (+ bias), X (M, K) and
// W (N, K) row-major (the Linear layers of the model behind model.forward, the in_proj /
// x_proj / dt_proj / out_proj of the Mamba blocks), all arithmetic in fp32 with
// v_mfma_f32_16x16x4_f32.
//
// Tiles. A workgroup (4 waves) owns a 128 x BN tile of Y (BN = 32 NJ: 128, 96 or 64) and
// walks K in steps of 16; the waves form a 2 x 2 grid of 64 x BN/2 sub-tiles, 4 NJ
// independent MFMA accumulator chains each. The X and W slices of a step go global -> LDS
// with the gfx950 buffer loads that write LDS directly (buffer_load_dwordx4 ... lds): no
// registers and no LDS store instructions. Each load moves one MFMA operand fragment: lane
// 16 q + i reads row i, k = 4 q .. 4 q + 3 of a 16 x 16 block, and the LDS receives the 64
// lanes' 16 bytes in lane order, so the fragment a wave later reads back with one
// ds_read_b128 per lane at lane * 16 is conflict-free. In MFMA t of a step lane group q
// supplies k = 4 q + t (the same permutation of k for both operands leaves the sum
// unchanged, and the order of the sum is fixed).
//
// Pipelining. Four LDS stages, each its own LDS object, three steps in flight: the loads of
// step s + 3 are issued before the MFMAs of step s. The compiler's wait counters tell the
// objects apart, so reading one stage does not wait for loads into the others; the loads are
// unconditional (steps past K are pushed out of range), which keeps those counts exact. One
// s_barrier per step, after the wave's loads of the next stage have landed.
//
// Edges. Each tile gets buffer descriptors that end with its last valid row, so rows past M
// read zeros and their stores are dropped; columns past N and k past K are pushed out of
// range with bit 31 of the per-lane offset. K % 4 == 0.
//
// Order. Workgroup b runs on XCD b % 8; consecutive tile ids are given to one XCD, and
// tiles are numbered in groups of 8 row tiles (a group walks its columns), so the tiles in
// flight on an XCD share X rows and W rows through that XCD's L2.
//
// Split K. When the tiles alone leave CUs idle (prompts of a few hundred tokens), K may be
// cut into S slices of a multiple of 16 (at least 128 each) and every (tile, slice) pair is
// a workgroup of its own (slice z of row tile tm is row tile tm + z mt of an S times taller
// grid, so the ordering above is unchanged); each writes its raw partial tile to a
// workspace (S, M, N), and a second kernel adds the S partials in slice order
// (deterministic) and applies the epilogue (row scale, bias, beta, gate) in the same order
// as the unsplit kernel. The tile width and S are chosen together by a cost model measured
// on MI355X: a CU running one of these workgroups does 0.44 TFLOP/s, two or more 0.50 (of
// 0.61 peak), the partials cost their bytes written and read at 5 TB/s, and the finishing
// launch about 4 us.
//
// Measured (MI355X, fp32 TFLOP/s, this kernel / hipBLASLt): M 32768 N 2048 K 4096 150 / 151,
// M 32768 N 8448 K 2016 148 / 149, M 8192 N 3072 K 768 119 / 118. At a clock of 2.4 GHz the
// fp32 MFMA peak is 157 TFLOP/s; with the operand loads running the clock drops to about
// 2.2-2.3 GHz (GRBM_GUI_ACTIVE over the dispatch time) and the MFMA pipe is busy 85-92% of
// the cycles (SQ_VALU_MFMA_BUSY_CYCLES).
#include <algorithm>

#include "common.hpp"
#include "glue.hpp"

namespace {

constexpr int BM = 128, BK = 16;
constexpr int GM = 8;             // row tiles per ordering group
constexpr int kFrag = 256;        // floats per 16 x 16 operand fragment
constexpr int kStage = 16 * kFrag;  // X (8 fragments) + W (8 fragments): 16 KB

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

struct GemmArgs {
    const float* X; long ldx;
    const float* W; long ldw;
    float* Y; long ldy;
    const float* bias;
    int M, N, K;
    float beta;
    int mt, nt;
    // row scale (RS): Y[m, :] = s[m] (X W^T)[m, :] + ..., s[m] = 1 / sqrt(inv_div *
    // sum_j ssq[m nssq + j] + eps) -- an RMSNorm of X's rows applied after the product
    const float* ssq; int nssq; float inv_div, eps;
    int gate_c0;   // columns >= gate_c0 (a multiple of 16) are stored as silu(value)
    // split K: ks slices of kslice (the last may be shorter); part (ks, M, N) row-major
    int ks, kslice;
    float* part;
};

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void to_lds(__amdgpu_buffer_rsrc_t r, float* lds, unsigned voff,
                                       unsigned soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voff, soff, 0, 0);
}

// End of a step: at most 8 of the wave's loads (the two younger stages) still in flight
// (vmcnt(8); expcnt and lgkmcnt at their maxima in the gfx9 encoding), then the workgroup
// barrier. The scheduling barriers keep the step's MFMAs above the wait (the compiler would
// otherwise hoist the wait and barrier over them and the loads would not overlap them).
__device__ __forceinline__ void end_step() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0f78);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

template <int NJ, bool BETA, bool RS, bool SPLIT = false>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(GemmArgs a) {
    constexpr int BN = 32 * NJ;
    static_assert(!SPLIT || (!BETA && !RS), "the split kernel stores raw partials");
    __shared__ float rs[RS ? BM : 1];
    __shared__ __attribute__((aligned(16))) float s0[kStage];
    __shared__ __attribute__((aligned(16))) float s1[kStage];
    __shared__ __attribute__((aligned(16))) float s2[kStage];
    __shared__ __attribute__((aligned(16))) float s3[kStage];

    // ---- tile of this workgroup: consecutive ids per XCD, groups of GM row tiles (with
    // split K, over the S times taller grid of (slice, row tile) pairs)
    const int mtv = SPLIT ? a.mt * a.ks : a.mt;
    const int T = mtv * a.nt;
    const int b = blockIdx.x;
    const int xcd = b & 7, per = T >> 3, rem = T & 7;
    const int id = xcd * per + min(xcd, rem) + (b >> 3);
    const int gsz = GM * a.nt;
    const int grp = id / gsz, gr = id - grp * gsz;
    const int gm = min(GM, mtv - grp * GM);
    const int tmv = grp * GM + gr % gm, tn = gr / gm;
    const int kz = SPLIT ? tmv / a.mt : 0, tm = SPLIT ? tmv - kz * a.mt : tmv;
    // this workgroup's k range [kbeg, kbeg + K)
    const int kbeg = SPLIT ? kz * a.kslice : 0;
    const int K = SPLIT ? min(a.kslice, a.K - kbeg) : a.K;

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, i16 = lane & 15;
    const int wm = w >> 1, wn = w & 1;

    const int m0 = tm * BM, n0 = tn * BN;
    const int rows = min(BM, a.M - m0), cols = min(BN, a.N - n0);
    const auto rx = ssm::rsrc(a.X + (long)m0 * a.ldx + kbeg,
                              (unsigned)(((long)(rows - 1) * a.ldx + K) * 4));
    const auto rw = ssm::rsrc(a.W + (long)n0 * a.ldw + kbeg,
                              (unsigned)(((long)(cols - 1) * a.ldw + K) * 4));

    // Loads of wave w in a step: X row blocks 2w, 2w + 1 and W row blocks 2w, 2w + 1 (W row
    // blocks past the tile's BN rows read nothing); lane (q, i16) reads row 16 rb + i16,
    // k = k0 + 4 q .. + 3, into fragment rb of the stage (X) or 8 + rb (W).
    unsigned ox[2], ow[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int r = 16 * (2 * w + u) + i16;
        ox[u] = (unsigned)(((long)r * a.ldx + 4 * q) * 4);
        ow[u] = (2 * w + u < 2 * NJ) ? (unsigned)(((long)r * a.ldw + 4 * q) * 4) : 0x80000000u;
    }
    // The step's k offset rides in the scalar offset. In the main loop every load is in
    // range and the per-lane offsets are fixed (no vector ALU work between the MFMAs); in the
    // tail, lanes whose k is past K (the last partial step, and the steps after it) get bit
    // 31 in their own offset, which alone puts them out of range.
    auto load = [&](float* s, int k0) {
        const unsigned kk = (unsigned)k0 * 4u;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            to_lds(rx, s + (2 * w + u) * kFrag, ox[u], kk);
            to_lds(rw, s + (8 + 2 * w + u) * kFrag, ow[u], kk);
        }
    };
    auto load_tail = [&](float* s, int k0) {
        const unsigned kk = (unsigned)min(k0, K) * 4u;
        const unsigned oor = k0 + 4 * q < K ? 0u : 0x80000000u;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            to_lds(rx, s + (2 * w + u) * kFrag, ox[u] | oor, kk);
            to_lds(rw, s + (8 + 2 * w + u) * kFrag, ow[u] | oor, kk);
        }
    };

    floatx4 acc[4][NJ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // 16 NJ MFMAs per step: X fragments 4 wm + i, W fragments NJ wn + j
    auto compute = [&](const float* s) {
        floatx4 xa[4], wb[NJ];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            xa[i] = *reinterpret_cast<const floatx4*>(s + (4 * wm + i) * kFrag + 4 * lane);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            wb[j] = *reinterpret_cast<const floatx4*>(s + (8 + NJ * wn + j) * kFrag + 4 * lane);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[i][j] = mfma4(xa[i][t], wb[j][t], acc[i][j]);
    };

    // Steps in blocks of four (one per stage): the main loop while every load of a block is
    // a whole step inside K, then the tail blocks with range-checked loads (a block that
    // runs past K computes on zeros).
    const int nk = (K + BK - 1) / BK;
    const int nfull = K / BK;   // steps that lie wholly inside K
    auto block = [&](int s, auto ld) {
        ld(s3, (s + 3) * BK);
        compute(s0);
        end_step();
        ld(s0, (s + 4) * BK);
        compute(s1);
        end_step();
        ld(s1, (s + 5) * BK);
        compute(s2);
        end_step();
        ld(s2, (s + 6) * BK);
        compute(s3);
        end_step();
    };
    if (nfull >= 3) {
        load(s0, 0);
        load(s1, BK);
        load(s2, 2 * BK);
    } else {
        load_tail(s0, 0);
        load_tail(s1, BK);
        load_tail(s2, 2 * BK);
    }
    end_step();
    int s = 0;
    for (; s + 7 <= nfull; s += 4) block(s, load);
    for (; s < nk; s += 4) block(s, load_tail);

    // ---- row scales of the tile's rows (partial sums added in order)
    if constexpr (RS) {
        if (threadIdx.x < BM) {
            float v = 1.f;
            if ((int)threadIdx.x < rows) {
                const float* p = a.ssq + (long)(m0 + threadIdx.x) * a.nssq;
                float sum = 0.f;
                for (int j = 0; j < a.nssq; ++j) sum += p[j];
                v = rsqrtf(sum * a.inv_div + a.eps);
            }
            rs[threadIdx.x] = v;
        }
        __syncthreads();
    }

    // ---- epilogue: acc[i][j][r] is Y[m0 + 16 (4 wm + i) + 4 q + r][n0 + 16 (NJ wn + j) + i16]
    if constexpr (SPLIT) {   // the raw partial tile of slice kz
        const auto rp = ssm::rsrc(a.part + ((long)kz * a.M + m0) * a.N + n0,
                                  (unsigned)(((long)(rows - 1) * a.N + cols) * 4));
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = 16 * (NJ * wn + j) + i16;
            const unsigned oor = c < cols ? 0u : 0x80000000u;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 16 * (4 * wm + i) + 4 * q + r;
                    ssm::bstore4(acc[i][j][r], rp, ((unsigned)(row * a.N + c) * 4u) | oor);
                }
        }
        return;
    }
    const auto ry = ssm::rsrc(a.Y + (long)m0 * a.ldy + n0,
                              (unsigned)(((long)(rows - 1) * a.ldy + cols) * 4));
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = 16 * (NJ * wn + j) + i16;
        const unsigned oor = c < cols ? 0u : 0x80000000u;
        const float bv = a.bias && c < cols ? a.bias[n0 + c] : 0.f;
        // the 16 columns of block j lie on one side of gate_c0: the choice is wave-uniform
        const bool gate = n0 + 16 * (NJ * wn + j) >= a.gate_c0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * (4 * wm + i) + 4 * q + r;
                const unsigned off = ((unsigned)(row * a.ldy + c) * 4u) | oor;
                float v = acc[i][j][r];
                if constexpr (RS) v *= rs[row];
                v += bv;
                if constexpr (BETA) v += a.beta * ssm::bload4(ry, off);
                if (gate) v = ssm::silu_fast(v);
                ssm::bstore4(v, ry, off);
            }
    }
}

// Split-K finish: Y = epilogue(sum over slices z = 0 .. ks-1 of part[z]), added in slice
// order; the epilogue in the unsplit kernel's order (row scale, bias, beta, gate). Thread
// (row m = blockIdx.y, columns 4 c4 .. 4 c4 + 3); N % 4 == 0.
__global__ __launch_bounds__(256) void gemm_finish_kernel(GemmArgs a) {
    const int m = blockIdx.y;
    const int c4 = blockIdx.x * 256 + threadIdx.x;
    if (4 * c4 >= a.N) return;
    const long MN = (long)a.M * a.N;
    const float4* p = reinterpret_cast<const float4*>(a.part + (long)m * a.N) + c4;
    float4 v = p[0];
    for (int z = 1; z < a.ks; ++z) {
        const float4 u = p[z * (MN / 4)];
        v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
    }
    float s = 1.f;
    if (a.ssq) {   // same order as the unsplit kernel's row scales
        const float* q = a.ssq + (long)m * a.nssq;
        float sum = 0.f;
        for (int j = 0; j < a.nssq; ++j) sum += q[j];
        s = rsqrtf(sum * a.inv_div + a.eps);
    }
    float* y = a.Y + (long)m * a.ldy + 4 * c4;
    float o[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int n = 4 * c4 + e;
        float t = o[e];
        if (a.ssq) t *= s;
        if (a.bias) t += a.bias[n];
        if (a.beta != 0.f) t += a.beta * y[e];
        if (n >= a.gate_c0) t = ssm::silu_fast(t);
        y[e] = t;
    }
}

// Column tile width: the one with the fewest rounds of 512 resident workgroups (two per
// CU), weighting a tile's cost by its width plus one (the X slice every tile loads).
int pick_nj(int M, int N) {
    const long mt = (M + BM - 1) / BM;
    int best = 4;
    double cost = 1e300;
    for (int nj : {4, 3, 2}) {
        const long t = mt * ((N + 32 * nj - 1) / (32 * nj));
        const double c = (double)((t + 511) / 512) * (nj + 1);
        if (c < cost - 1e-9) cost = c, best = nj;
    }
    return best;
}

template <int NJ>
void launch_nj(const GemmArgs& a, bool beta, hipStream_t st) {
    const dim3 block(256);
    if (a.ks > 1) {
        gemm_f32_kernel<NJ, false, false, true><<<dim3((unsigned)(a.mt * a.ks * a.nt)), block,
                                                  0, st>>>(a);
        gemm_finish_kernel<<<dim3((unsigned)((a.N / 4 + 255) / 256), (unsigned)a.M), block, 0,
                             st>>>(a);
        return;
    }
    const dim3 grid((unsigned)(a.mt * a.nt));
    if (a.ssq) {
        if (beta) gemm_f32_kernel<NJ, true, true><<<grid, block, 0, st>>>(a);
        else gemm_f32_kernel<NJ, false, true><<<grid, block, 0, st>>>(a);
    } else {
        if (beta) gemm_f32_kernel<NJ, true, false><<<grid, block, 0, st>>>(a);
        else gemm_f32_kernel<NJ, false, false><<<grid, block, 0, st>>>(a);
    }
}

// ---------------------------------------------------------------- x_proj -> dt_proj
// The Mamba-1 block's projections between the conv and the scan in one pass over xc:
//   dbl = xc Wx^T           (T, R + 2N): dt_low | B | C, the scan's B and C operands
//   dt  = dt_low Wdt^T      (T, D), the scan's dt before its bias and softplus, or, given
//                           the bias, dt' = softplus(dt + bias) itself
// A workgroup (8 waves) owns 32 rows (time steps). x_proj: wave w sums its eighth of K for
// the 2 x NCB 16 x 16 tiles of the rows' dbl, with operand fragments read from global
// memory straight into registers (one b128 per lane) through a ring of PD k blocks in
// flight; the eight partial tiles meet in LDS and are added in wave order. dt_low stays in
// LDS, in MFMA operand order, as the A operand of dt_proj; wave w then produces its share of
// dt's 16-column blocks (K = R, Wdt from L2 in groups of column blocks). xc is read once and
// dt_low never reaches memory. Loads and steps past a wave's range are issued anyway with
// out-of-range offsets (they read zeros and their stores are dropped), so every wave runs
// the same straight-line ring and the compiler's wait counts stay exact.
constexpr int XD_ROWS = 32;
constexpr int XD_WAVES = 8;

struct XdArgs {
    const float* x; long ldx;       // xc (T, D)
    const float* Wx;                // (RN, D) row-major
    const float* Wdt;               // (D, R) row-major
    float* dbl; long lddbl;         // (T, RN)
    float* dt; long lddt;           // (T, D)
    int T, D, R, RN;
    const float* dtb;               // given: dt = softplus(dt_low Wdt^T + dtb)
};

template <int NCB, int KB2, int PD>
__global__ __launch_bounds__(XD_ROWS * 16, 1) void xproj_dt_kernel(XdArgs a) {
    __shared__ __attribute__((aligned(16))) float red[XD_WAVES][2 * NCB][kFrag];
    __shared__ __attribute__((aligned(16))) float dl[2 * KB2][kFrag];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, i16 = lane & 15;
    const int row0 = blockIdx.x * XD_ROWS;
    const int rows = min(XD_ROWS, a.T - row0);

    for (int e = threadIdx.x; e < 2 * KB2 * kFrag; e += blockDim.x) (&dl[0][0])[e] = 0.f;

    // ---- x_proj, wave w: k blocks [kb0, kb0 + per), those at or past nkb read nothing
    const int nkb = (a.D + 15) / 16;
    const int per = (nkb + XD_WAVES - 1) / XD_WAVES;
    const int kb0 = w * per;
    const auto rx = ssm::rsrc(a.x + (long)row0 * a.ldx, (unsigned)(((long)(rows - 1) * a.ldx + a.D) * 4));
    const auto rwx = ssm::rsrc(a.Wx, (unsigned)(((long)(a.RN - 1) * a.D + a.D) * 4));
    unsigned oxr[2], owr[NCB];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) oxr[rb] = (unsigned)(((long)(16 * rb + i16) * a.ldx + 4 * q) * 4);
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) owr[cb] = (unsigned)(((long)(16 * cb + i16) * a.D + 4 * q) * 4);

    floatx4 acc[2][NCB];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) acc[rb][cb] = floatx4{0.f, 0.f, 0.f, 0.f};
    floatx4 fx[PD][2], fw[PD][NCB];
    auto fetch = [&](int buf, int kb) {
        const int k = 16 * kb + 4 * q;
        const bool ok = kb < kb0 + per && k < a.D;
        const unsigned oor = ok ? 0u : 0x80000000u;
        const unsigned kk = ok ? (unsigned)kb * 64u : 0u;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) fx[buf][rb] = ssm::bload16<floatx4>(rx, (oxr[rb] | oor) + kk);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) fw[buf][cb] = ssm::bload16<floatx4>(rwx, (owr[cb] | oor) + kk);
    };
    auto step = [&](int buf) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
                    acc[rb][cb] = mfma4(fx[buf][rb][t], fw[buf][cb][t], acc[rb][cb]);
    };
#pragma unroll
    for (int u = 0; u < PD - 1; ++u) fetch(u, kb0 + u);
    for (int kb = kb0; kb < kb0 + per; kb += PD) {
#pragma unroll
        for (int u = 0; u < PD; ++u) {
            // the scheduling barriers keep each refill ahead of the MFMAs it overlaps (the
            // scheduler would otherwise sink the loads next to their use)
            fetch((u + PD - 1) % PD, kb + u + PD - 1);
            __builtin_amdgcn_sched_barrier(0);
            step(u);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
            *reinterpret_cast<floatx4*>(&red[w][rb * NCB + cb][4 * lane]) = acc[rb][cb];
    __syncthreads();

    // ---- the eight partial tiles, added in wave order: element f of tile (rb, cb) is row
    // 16 rb + 4 (l / 16) + r, column 16 cb + l % 16 with l = f / 4, r = f % 4
    const auto rdb = ssm::rsrc(a.dbl + (long)row0 * a.lddbl, (unsigned)(((long)(rows - 1) * a.lddbl + a.RN) * 4));
    for (int e = threadIdx.x; e < 2 * NCB * kFrag; e += blockDim.x) {
        const int tile = e / kFrag, f = e % kFrag;
        const int rb = tile / NCB, cb = tile % NCB;
        float v = 0.f;
#pragma unroll
        for (int ww = 0; ww < XD_WAVES; ++ww) v += red[ww][tile][f];
        const int l = f >> 2, r = f & 3;
        const int row = 16 * rb + 4 * (l >> 4) + r, col = 16 * cb + (l & 15);
        if (col < a.RN) ssm::bstore4(v, rdb, (unsigned)(row * a.lddbl + col) * 4u);
        if (col < a.R) {
            // A operand of dt_proj: fragment (rb, k block col / 16), lane 16 (col % 16 / 4) +
            // row % 16, component col % 4
            const int kb2 = col >> 4, cq = (col & 15) >> 2, ct = col & 3;
            dl[rb * KB2 + kb2][(cq * 16 + (row & 15)) * 4 + ct] = v;
        }
    }
    __syncthreads();

    // ---- dt_proj, wave w: 16-column blocks [cb0, cb0 + cper) of dt
    floatx4 xa[2][KB2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int kb = 0; kb < KB2; ++kb)
            xa[rb][kb] = *reinterpret_cast<const floatx4*>(&dl[rb * KB2 + kb][4 * lane]);
    const int ndb = (a.D + 15) / 16;
    const int cper = (ndb + XD_WAVES - 1) / XD_WAVES;
    const int cb0 = w * cper;
    const auto rwd = ssm::rsrc(a.Wdt, (unsigned)(((long)(a.D - 1) * a.R + a.R) * 4));
    const auto rdt = ssm::rsrc(a.dt + (long)row0 * a.lddt, (unsigned)(((long)(rows - 1) * a.lddt + a.D) * 4));
    unsigned owd[KB2];
#pragma unroll
    for (int kb = 0; kb < KB2; ++kb)
        owd[kb] = (16 * kb + 4 * q < a.R) ? (unsigned)((i16 * a.R + 16 * kb + 4 * q) * 4) : 0x80000000u;
    // Wdt fragments in groups of DG column blocks, all of a group loaded before any of its
    // outputs is stored: a load issued after stores counts as done only once those stores
    // are (one in-order counter), so a ring refilled between the stores would wait for them
    constexpr int DG = KB2 <= 3 ? 6 : 4;
    floatx4 wd[DG][KB2];
    auto wfetch = [&](int buf, int cb) {
        const bool ok = cb < cb0 + cper;
        const unsigned rr = (unsigned)(16 * cb * a.R) * 4u;
#pragma unroll
        for (int kb = 0; kb < KB2; ++kb)
            wd[buf][kb] = ssm::bload16<floatx4>(rwd, ok ? owd[kb] + rr : 0x80000000u);
    };
    auto out = [&](int buf, int cb) {
        floatx4 o[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int kb = 0; kb < KB2; ++kb)
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) o[rb] = mfma4(xa[rb][kb][t], wd[buf][kb][t], o[rb]);
        const int c = 16 * cb + i16;
        const bool live = cb < cb0 + cper && c < a.D;
        const unsigned oor = live ? 0u : 0x80000000u;
        const float bias = (a.dtb && live) ? a.dtb[c] : 0.f;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float v = a.dtb ? ssm::softplus_sel(o[rb][r] + bias) : o[rb][r];
                ssm::bstore4(v, rdt, ((unsigned)((16 * rb + 4 * q + r) * a.lddt + c) * 4u) | oor);
            }
    };
    for (int cb = cb0; cb < cb0 + cper; cb += DG) {
#pragma unroll
        for (int u = 0; u < DG; ++u) wfetch(u, cb + u);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < DG; ++u) out(u, cb + u);
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int NCB, int KB2>
void launch_xd(const XdArgs& a, hipStream_t st) {
    constexpr int PD = NCB <= 5 ? 4 : 3;
    const dim3 grid((unsigned)((a.T + XD_ROWS - 1) / XD_ROWS)), block(XD_ROWS * 16);
    xproj_dt_kernel<NCB, KB2, PD><<<grid, block, 0, st>>>(a);
}

template <int NCB>
void launch_xd_k(const XdArgs& a, int kb2, hipStream_t st) {
    switch (kb2) {
        case 1: launch_xd<NCB, 1>(a, st); break;
        case 2: launch_xd<NCB, 2>(a, st); break;
        case 3: launch_xd<NCB, 3>(a, st); break;
        default: launch_xd<NCB, 4>(a, st); break;
    }
}

}  // namespace

namespace ssm {

bool xproj_dt_ok(int T, int D, int R, int N, long ldx, long lddbl, long lddt) {
    const int RN = R + 2 * N;
    if (T <= 0 || D <= 0 || R <= 0 || N <= 0) return false;
    if (D % 4 || R % 4 || R > 64 || RN > 128) return false;
    if (ldx < D || ldx % 4 || lddbl < RN || lddt < D) return false;
    const long lim = 1L << 31;
    return (long)XD_ROWS * std::max({ldx, lddbl, lddt}) * 4 < lim && (long)RN * D * 4 < lim &&
           (long)D * R * 4 < lim;
}

ssm_status launch_xproj_dt(const float* x, long ldx, const float* Wx, const float* Wdt,
                           float* dbl, long lddbl, float* dt, long lddt, int T, int D, int R,
                           int N, hipStream_t st, const float* dt_bias) {
    if (!xproj_dt_ok(T, D, R, N, ldx, lddbl, lddt))
        return fail(SSM_ERR_INVALID_ARG, "xproj_dt: unsupported shape T %d D %d R %d N %d", T, D,
                    R, N);
    if (((uintptr_t)x | (uintptr_t)Wx | (uintptr_t)Wdt) & 15)
        return fail(SSM_ERR_INVALID_ARG, "xproj_dt: x, Wx, Wdt must be 16-byte aligned");
    XdArgs a{x, ldx, Wx, Wdt, dbl, lddbl, dt, lddt, T, D, R, R + 2 * N, dt_bias};
    // x_proj column tiles: 3, 4, 5, 6 or 8 (7 runs as 8; the extra tile reads zeros)
    const int ncb = (a.RN + 15) / 16, kb2 = (R + 15) / 16;
    if (ncb <= 3) launch_xd_k<3>(a, kb2, st);
    else if (ncb == 4) launch_xd_k<4>(a, kb2, st);
    else if (ncb == 5) launch_xd_k<5>(a, kb2, st);
    else if (ncb == 6) launch_xd_k<6>(a, kb2, st);
    else launch_xd_k<8>(a, kb2, st);
    return check_launch("xproj_dt");
}

bool gemm_ok(int M, int N, int K, long ldx, long ldw, long ldy) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 4) return false;
    if (ldx < K || ldw < K || ldy < N || ldx % 4 || ldw % 4) return false;
    // 32-bit offsets inside one tile's descriptors, bit 31 free for the range trick
    const long lim = 1L << 31;
    return (long)BM * ldx * 4 + (long)K * 4 < lim && (long)BM * ldw * 4 + (long)K * 4 < lim &&
           (long)BM * ldy * 4 < lim;
}

// Tile width and split of K for a grid under two rounds of resident workgroups (pick_nj's
// grid has fewer than 512 tiles): the (NJ, slice count) pair with the least modelled time
// (above), slices at least 128 deep and a multiple of 16, within the workspace
// (part_floats floats). Larger grids keep pick_nj's width, unsplit.
struct Plan { int nj, ks, kslice; };
Plan pick_plan(int M, int N, int K, size_t part_floats) {
    const long mt = (M + BM - 1) / BM;
    Plan p{pick_nj(M, N), 1, K};
    if (mt * ((N + 32 * p.nj - 1) / (32 * p.nj)) >= 512) return p;
    auto busy = [&](long wgs, int bn, int depth) {   // the most loaded CU's time (s)
        const long n = (wgs + 255) / 256;
        return (double)n * 2.0 * BM * bn * depth / (n == 1 ? 0.44e12 : 0.50e12);
    };
    double best = 1e300;
    for (int nj : {2, 3, 4}) {
        const int bn = 32 * nj;
        const long tiles = mt * ((N + bn - 1) / bn);
        const double t1 = busy(tiles, bn, K);
        if (t1 < best) best = t1, p = Plan{nj, 1, K};
        if (tiles >= 256 || N % 4 || K < 256) continue;
        for (int ks = 2; ks <= K / 128; ++ks) {
            if ((size_t)ks * M * N > part_floats) break;
            const int sl = ((K + ks - 1) / ks + 15) / 16 * 16;
            if ((K + sl - 1) / sl != ks) continue;
            const double t = busy(tiles * ks, bn, sl) + 8.0 * ks * M * N / 5e12 + 4e-6;
            if (t < best) best = t, p = Plan{nj, ks, sl};
        }
    }
    return p;
}

size_t gemm_split_floats(int M, int N, int K) {
    const Plan p = pick_plan(M, N, K, (size_t)-1);
    return p.ks > 1 ? (size_t)p.ks * M * N : 0;
}

ssm_status launch_gemm(const float* X, long ldx, const float* W, long ldw, const float* bias,
                       float* Y, long ldy, int M, int N, int K, float beta, hipStream_t st,
                       const float* ssq, int nssq, float inv_div, float eps, int gate_c0,
                       float* part, size_t part_floats) {
    if (!gemm_ok(M, N, K, ldx, ldw, ldy))
        return fail(SSM_ERR_INVALID_ARG, "gemm: unsupported shape M %d N %d K %d ld %ld/%ld/%ld",
                    M, N, K, ldx, ldw, ldy);
    if (((uintptr_t)X | (uintptr_t)W) & 15)
        return fail(SSM_ERR_INVALID_ARG, "gemm: X and W must be 16-byte aligned");
    // with a workspace, the width and split of pick_plan; without, pick_nj's width unsplit
    const bool ws = part && ((uintptr_t)part & 15) == 0;
    const Plan p = ws ? pick_plan(M, N, K, part_floats) : Plan{pick_nj(M, N), 1, K};
    const int nj = p.nj;
    GemmArgs a{X, ldx, W, ldw, Y, ldy, bias, M, N, K, beta, (M + BM - 1) / BM,
               (N + 32 * nj - 1) / (32 * nj), ssq, nssq, inv_div, eps, gate_c0, p.ks, p.kslice,
               p.ks > 1 ? part : nullptr};
    if (gate_c0 < N && gate_c0 % 16)
        return fail(SSM_ERR_INVALID_ARG, "gemm: gate column %d not a multiple of 16", gate_c0);
    if (ssq && nssq <= 0) return fail(SSM_ERR_INVALID_ARG, "gemm: row scale needs nssq > 0");
    if ((long)a.mt * a.nt > (1L << 30)) return fail(SSM_ERR_INVALID_ARG, "gemm: too many tiles");
    const bool bt = beta != 0.f;
    if (nj == 4) launch_nj<4>(a, bt, st);
    else if (nj == 3) launch_nj<3>(a, bt, st);
    else launch_nj<2>(a, bt, st);
    return check_launch("gemm_f32");
}

}  // namespace ssm

extern "C" ssm_status ssm_linear(const float* x, long ldx, const float* W, long ldw,
                                 const float* bias, float* y, long ldy, int M, int N, int K,
                                 float beta, void* stream) {
    SSM_REQUIRE(x && W && y, "ssm_linear: null x/W/y");
    SSM_REQUIRE(M >= 0 && N >= 0 && K > 0, "ssm_linear: bad shape");
    if (M == 0 || N == 0) return SSM_OK;
    return ssm::launch_gemm(x, ldx, W, ldw, bias, y, ldy, M, N, K, beta, (hipStream_t)stream);
}

extern "C" ssm_status ssm_m1_xproj_dt(const float* x, long ldx, const float* Wx, const float* Wdt,
                                      float* dbl, long lddbl, float* dt, long lddt, int T, int D,
                                      int R, int N, void* stream) {
    SSM_REQUIRE(x && Wx && Wdt && dbl && dt, "ssm_m1_xproj_dt: null pointer");
    if (T == 0) return SSM_OK;
    return ssm::launch_xproj_dt(x, ldx, Wx, Wdt, dbl, lddbl, dt, lddt, T, D, R, N,
                                (hipStream_t)stream);
}
