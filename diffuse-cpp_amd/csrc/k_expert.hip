// k_expert.hip — grouped Q4_K expert products on MFMA (gfx950).
//
// Computes the routed experts of src/diffuse-moe-graph.cpp:264-269 (ggml's
// mul_mat_id over Q4_K weights with Q8_K activations) and the shared expert of
// :280-286 (F32 activations), as one persistent launch per phase:
//   phase 0: h = silu(W_gate x) * (W_up x)       (gate and up of the same rows)
//   phase 1: y = W_down h
// (the conversion of h to the activation layout runs in between, k_prep.hip).
//
// Arithmetic.  Per 256-value super-block, a Q4_K row is  w = d*sc_j*q - dmin*m_j
// (j = 32-value sub-block).  With activations a (Q8_K quants, or scaled f32
// for the shared expert):
//   sum_k w a = d * S1 - dmin * S2,   S1 = sum_k (sc_j q) a,   S2 = sum_j m_j sum_{k in j} a
// sc_j*q <= 945 and the Q8_K quants are integers, all exact in f16, so
// v_mfma_f32_16x16x32_f16 gives S1 as an exact integer dot (f32 accumulation of
// exact products); S2 uses v_mfma_f32_16x16x16_f16 on the 16-value sums.  The
// super-block result is scaled by the activation scale and accumulated in f32.
//
// Operand layout (checked on the hardware): srcA lane l = activation row l%16,
// k = 8*(l/16)+e; srcB lane l = weight row l%16, same k; D lane l = weight row
// l%16, activation rows 4*(l/16)+i.  Lane group g = l/16 handles the 32 qs
// bytes of Q4_K chunk g (sub-blocks 2g, 2g+1); MFMA step s takes qs dword s.
// A nibble q becomes the f16 1024+q (or 1024+16q for the high nibble) by OR-ing
// it into the mantissa of 1024.0, and one packed fma subtracts the offset and
// applies sc exactly: (1024+q)*sc - 1024*sc = q*sc.
//
// Memory.  Weights are in the tiled layout (k_quant.hip: 16-row tiles,
// super-block-major), so a tile's super-block is one contiguous 2304-byte run
// and every weight load of a wave is coalesced.  A workgroup's four waves work
// on the same 16 activation rows (one expert's chunk of pairs, or 8 tokens of
// the shared expert) and different weight tiles; the activation tile of each
// super-block is loaded once per workgroup into double-buffered LDS while the
// previous super-block is computed.
#include "dmoe_internal.h"

namespace dmoe {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int WAVES = 4;                 // waves per workgroup
constexpr int RT = 2;                    // 16-row weight tiles per wave
constexpr int GROWS_GU = WAVES * 16;     // weight rows of a gate/up item (gate and up)
constexpr int GROWS_DN = WAVES * 16 * RT;    // weight rows of a down item
#ifndef DMOE_X_BLOCKS
#define DMOE_X_BLOCKS 1024               // persistent grid
#endif
constexpr int A_ROW = 264;               // f16 per LDS activation row (256 + pad)
constexpr int TILE_BYTES = 16 * Q4K_BYTES;   // one tile x one super-block

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ float h16f(uint32_t u) { return (float)__builtin_bit_cast(_Float16, (uint16_t)u); }

struct Q4KTile {        // a lane's share of one 16-row tile in one super-block
    uint4 h;            // d, dmin, scales[12]
    uint4 q0, q1;       // qs bytes 32g .. 32g+31
};

// tile: base of the tile's super-block runs; lane row r16, group g
__device__ __forceinline__ void load_tile(Q4KTile &t, const uint8_t *tile, int sb, int r16, int g)
{
    const uint8_t *blk = tile + (size_t)sb * TILE_BYTES + r16 * Q4K_BYTES;
    t.h = *reinterpret_cast<const uint4 *>(blk);
    const uint4 *qp = reinterpret_cast<const uint4 *>(blk + 16 + 32 * g);
    t.q0 = qp[0];
    t.q1 = qp[1];
}

struct Q4KOps {
    h8 b[8];            // srcB of the 8 MFMA steps
    h4 bm;              // srcB of the min term: m_2g, m_2g, m_2g+1, m_2g+1
    float d, dmin;
};

__device__ __forceinline__ void dequant_tile(const Q4KTile &t, int g, Q4KOps &o)
{
    // 6-bit scale / min of sub-blocks 2g and 2g+1 (bytes jj, jj+1 of each word)
    const uint32_t shift = 16u * (uint32_t)(g & 1);
    const uint32_t by = (t.h.y >> shift) & 0xffffu;
    const uint32_t bz = (t.h.z >> shift) & 0xffffu;
    const uint32_t bw = (t.h.w >> shift) & 0xffffu;
    uint32_t sc0, sc1, m0, m1;
    if (g < 2) {
        sc0 = by & 63u;
        sc1 = (by >> 8) & 63u;
        m0 = bz & 63u;
        m1 = (bz >> 8) & 63u;
    } else {
        sc0 = (bw & 15u) | (((by >> 6) & 3u) << 4);
        sc1 = ((bw >> 8) & 15u) | (((by >> 14) & 3u) << 4);
        m0 = ((bw >> 4) & 15u) | (((bz >> 6) & 3u) << 4);
        m1 = ((bw >> 12) & 15u) | (((bz >> 14) & 3u) << 4);
    }
    o.d = h16f(t.h.x & 0xffffu);
    o.dmin = h16f(t.h.x >> 16);
    const _Float16 a0 = (_Float16)(float)sc0, n0 = (_Float16)(-1024.0f * (float)sc0);
    const _Float16 a1 = (_Float16)((float)sc1 * 0.0625f), n1 = (_Float16)(-64.0f * (float)sc1);
    const h2 SC0 = {a0, a0}, N0 = {n0, n0}, SC1 = {a1, a1}, N1 = {n1, n1};
    const uint32_t q[8] = {t.q0.x, t.q0.y, t.q0.z, t.q0.w, t.q1.x, t.q1.y, t.q1.z, t.q1.w};
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const uint32_t w = q[s], w8 = w >> 8;
        const h2 lo02 = __builtin_elementwise_fma(as_h2((w & 0x000F000Fu) | 0x64006400u), SC0, N0);
        const h2 lo13 = __builtin_elementwise_fma(as_h2((w8 & 0x000F000Fu) | 0x64006400u), SC0, N0);
        const h2 hi02 = __builtin_elementwise_fma(as_h2((w & 0x00F000F0u) | 0x64006400u), SC1, N1);
        const h2 hi13 = __builtin_elementwise_fma(as_h2((w8 & 0x00F000F0u) | 0x64006400u), SC1, N1);
        o.b[s] = (h8){lo02.x, lo02.y, lo13.x, lo13.y, hi02.x, hi02.y, hi13.x, hi13.y};
    }
    const _Float16 fm0 = (_Float16)(float)m0, fm1 = (_Float16)(float)m1;
    o.bm = (h4){fm0, fm0, fm1, fm1};
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// One super-block of the 16 activation rows of a work item, in LDS.
struct ATile {
    uint16_t v[16][A_ROW];      // f16 values in operand order (row padded)
    uint16_t bs[16][16];        // sums of 16
    float d[16];                // per-row super-block scale
};

// A thread's share of the per-super-block copy of the activation tile into LDS:
// value pieces p0 = tid, p1 = tid + 256 (row p/32, 16-byte column p%32), the
// bs piece for tid < 32 (row tid/2, half tid%2), the scale for tid in 32..47.
struct AFeed {
    int rv0, rv1, rbs, rd;      // activation rows (global) of those pieces
    uint4 v0, v1, bs;
    float d;
};

__device__ __forceinline__ void feed_load(AFeed &f, const ActMfma &act, int sb, int tid)
{
    // every thread issues the same four loads (pieces it does not store read
    // valid addresses), so the loads of a pipeline step are branch-free and
    // the compiler's load counting keeps the next steps in flight
    const int K = act.K, nsb = K / 256;
    f.v0 = *reinterpret_cast<const uint4 *>(act.v + (size_t)f.rv0 * K + sb * 256 + (tid & 31) * 8);
    f.v1 = *reinterpret_cast<const uint4 *>(act.v + (size_t)f.rv1 * K + sb * 256 + (tid & 31) * 8);
    f.bs = *reinterpret_cast<const uint4 *>(act.bs + (size_t)f.rbs * (K / 16) + sb * 16 + (tid & 1) * 8);
    f.d = act.d[(size_t)f.rd * nsb + sb];
}

__device__ __forceinline__ void feed_store(const AFeed &f, ATile &a, int tid)
{
    *reinterpret_cast<uint4 *>(&a.v[tid >> 5][(tid & 31) * 8]) = f.v0;
    *reinterpret_cast<uint4 *>(&a.v[(tid >> 5) + 8][(tid & 31) * 8]) = f.v1;
    if (tid < 32)
        *reinterpret_cast<uint4 *>(&a.bs[tid >> 1][(tid & 1) * 8]) = f.bs;
    else if (tid < 48)
        a.d[tid - 32] = f.d;
}

// One super-block: R weight tiles against the activation tile a.
template <int R>
__device__ __forceinline__ void compute_sb(const Q4KTile (&cur)[R], const ATile &a, int r16, int g,
                                           float (&acc)[R][4])
{
    const float4 dxv = *reinterpret_cast<const float4 *>(&a.d[4 * g]);
    const float dx[4] = {dxv.x, dxv.y, dxv.z, dxv.w};
    const h4 ab = __builtin_bit_cast(h4, *reinterpret_cast<const uint2 *>(&a.bs[r16][4 * g]));
#pragma unroll
    for (int r = 0; r < R; r++) {
        Q4KOps o;
        dequant_tile(cur[r], g, o);
        f4 s1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const h8 av = __builtin_bit_cast(
                h8, *reinterpret_cast<const uint4 *>(&a.v[r16][g * 64 + s * 8]));
            s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, o.b[s], s1, 0, 0, 0);
        }
        f4 s2 = {0.0f, 0.0f, 0.0f, 0.0f};
        s2 = __builtin_amdgcn_mfma_f32_16x16x16f16(ab, o.bm, s2, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[r][i] += dx[i] * (o.d * s1[i] - o.dmin * s2[i]);
    }
}

// One pipeline step: super-block s is computed from cur (skipped past the last
// super-block) while the weights of s + 1 load into nxt and the activations of
// s + 1 into the other LDS buffer.  Indices are clamped to the last
// super-block, whose repeated loads hit the cache, so that every step issues
// the same loads.
template <int R>
__device__ __forceinline__ void step_sb(const Q4KTile (&cur)[R], Q4KTile (&nxt)[R],
                                        const uint8_t *const (&tile)[R], const ActMfma &act,
                                        AFeed &feed, ATile (&sa)[2], int s, int nsb, int tid,
                                        int r16, int g, float (&acc)[R][4])
{
    const int sn = min(s + 1, nsb - 1);
    feed_load(feed, act, sn, tid);
#pragma unroll
    for (int r = 0; r < R; r++) load_tile(nxt[r], tile[r], sn, r16, g);
    if (s < nsb) compute_sb<R>(cur, sa[s & 1], r16, g, acc);
    if (s + 1 < nsb) feed_store(feed, sa[(s + 1) & 1], tid);
    __syncthreads();
}

// Accumulate R weight tiles (tile[r]: base of the tile's super-block runs)
// against the item's 16 activation rows, all super-blocks.
template <int R>
__device__ __forceinline__ void run_item(const uint8_t *const (&tile)[R], const ActMfma &act,
                                         AFeed &feed, ATile (&sa)[2], int tid, int r16, int g,
                                         float (&acc)[R][4])
{
    const int nsb = act.K / 256;
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[r][i] = 0.0f;
    Q4KTile t0[R], t1[R];
    feed_load(feed, act, 0, tid);
#pragma unroll
    for (int r = 0; r < R; r++) load_tile(t0[r], tile[r], 0, r16, g);
    feed_store(feed, sa[0], tid);
    __syncthreads();
    for (int sb = 0; sb < nsb; sb += 2) {
        step_sb<R>(t0, t1, tile, act, feed, sa, sb, nsb, tid, r16, g, acc);
        step_sb<R>(t1, t0, tile, act, feed, sa, sb + 1, nsb, tid, r16, g, acc);
    }
}

// Workgroup items of phase 0: routed (work-list entry ec, group of 64 rows),
// then shared (chunk of 8 tokens, group of 64 rows); phase 1 the same with
// groups of 128 rows.  A routed item's 16 activation rows are the pairs of its
// entry (one expert, up to 16 consecutive pairs of it); a shared item's are the
// hi / lo halves of its 8 tokens' split activations interleaved (t hi, t lo,
// ...), so that each lane's four outputs are (t, hi), (t, lo), (t+1, hi),
// (t+1, lo) and the halves are summed in-lane.
template <int PHASE>
__global__ __launch_bounds__(WAVES * 64) void k_expert_q4k(MoeJob job)
{
    constexpr bool DOWN = PHASE == 1;
    constexpr int GROWS = DOWN ? GROWS_DN : GROWS_GU;
    __shared__ ATile sa[2];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int N = job.n_tokens, K = job.top_k;
    const int H = job.H, FF = job.FF, SF = job.SF;
    const int n_ec = job.wl.n_ec[0];
    const int nch = job.has_shared ? (N + SHARED_CHUNK - 1) / SHARED_CHUNK : 0;
    const int rg = (DOWN ? H : FF) / GROWS, rg_sh = (DOWN ? H : SF) / GROWS;
    const int routed_items = n_ec * rg;
    const int total = routed_items + nch * rg_sh;
    const int nsbH = H / 256, nsbF = FF / 256, nsbS = SF / 256;

    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        const bool shared = item >= routed_items;
        const int j = shared ? item - routed_items : item;
        const int rgn = shared ? rg_sh : rg;
        const int unit = j / rgn;                 // work-list entry or shared chunk
        const int row0 = (j - unit * rgn) * GROWS + wave * (GROWS / WAVES);
        int t_first, nt, e = 0;
        if (!shared) {
            e = job.wl.ec_expert[unit];
            const int c0 = job.wl.ec_chunk[unit] * EXPERT_CHUNK;
            t_first = job.offsets[e] + c0;
            nt = min(EXPERT_CHUNK, job.counts[e] - c0);
        } else {
            t_first = unit * SHARED_CHUNK;
            nt = min(SHARED_CHUNK, N - t_first);
        }
        // activation row of item row jr (0..15): tokens in phase 0, pairs in
        // phase 1; shared rows interleave hi and lo (lo rows start at N)
        auto arow = [&](int jr) {
            if (shared) return t_first + min(jr >> 1, nt - 1) + (jr & 1) * N;
            const int p = job.perm[t_first + min(jr, nt - 1)];
            return DOWN ? p : p / K;
        };
        AFeed feed;
        feed.rv0 = arow(tid >> 5);
        feed.rv1 = arow((tid >> 5) + 8);
        feed.rbs = arow((tid >> 1) & 15);
        feed.rd = arow(tid >= 32 && tid < 48 ? tid - 32 : 0);

        const uint8_t *tile[RT];
        if (!DOWN) {
            const WTensor &a = shared ? job.sg : job.eg;
            const WTensor &b = shared ? job.su : job.eu;
            tile[0] = a.data + (size_t)e * a.nb2 + (size_t)(row0 / 16) * nsbH * TILE_BYTES;
            tile[1] = b.data + (size_t)e * b.nb2 + (size_t)(row0 / 16) * nsbH * TILE_BYTES;
        } else {
            const WTensor &a = shared ? job.sd : job.ed;
            const int n = shared ? nsbS : nsbF;
#pragma unroll
            for (int r = 0; r < RT; r++)
                tile[r] = a.data + (size_t)e * a.nb2 + (size_t)(row0 / 16 + r) * n * TILE_BYTES;
        }
        const ActMfma &act = DOWN ? (shared ? job.ahs : job.ah) : (shared ? job.axs : job.ax);
        float acc[RT][4];
        run_item<RT>(tile, act, feed, sa, tid, r16, g, acc);

        if (!shared) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (4 * g + i >= nt) continue;
                const int p = job.perm[t_first + 4 * g + i];
                if (!DOWN) {
                    job.h[(size_t)p * FF + row0 + r16] = silu(acc[0][i]) * acc[1][i];
                } else {
                    float *o = job.ye + (size_t)p * H + row0 + r16;
#pragma unroll
                    for (int r = 0; r < RT; r++) o[16 * r] = acc[r][i];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                if (2 * g + (i >> 1) >= nt) continue;
                const int t = t_first + 2 * g + (i >> 1);
                if (!DOWN) {
                    job.hs[(size_t)t * SF + row0 + r16] =
                        silu(acc[0][i] + acc[0][i + 1]) * (acc[1][i] + acc[1][i + 1]);
                } else {
                    float *o = job.ys + (size_t)t * H + row0 + r16;
#pragma unroll
                    for (int r = 0; r < RT; r++) o[16 * r] = acc[r][i] + acc[r][i + 1];
                }
            }
        }
    }
}

int expert_rows_per_item(int phase) { return phase == 0 ? GROWS_GU : GROWS_DN; }

hipError_t launch_expert_q4k(int phase, const MoeJob &job, hipStream_t s)
{
    if (job.FF % GROWS_GU || job.FF % 256 || job.H % GROWS_DN || job.H % 256 ||
        job.ax.K != job.H || job.ah.K != job.FF ||
        (job.has_shared && (job.SF % GROWS_GU || job.SF % 256 || job.ahs.K != job.SF)))
        return hipErrorInvalidValue;
    if (phase == 0)
        hipLaunchKernelGGL(k_expert_q4k<0>, dim3(DMOE_X_BLOCKS), dim3(WAVES * 64), 0, s, job);
    else
        hipLaunchKernelGGL(k_expert_q4k<1>, dim3(DMOE_X_BLOCKS), dim3(WAVES * 64), 0, s, job);
    return hipGetLastError();
}

} // namespace dmoe
