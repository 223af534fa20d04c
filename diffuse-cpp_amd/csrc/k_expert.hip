// k_expert.hip — grouped Q4_K expert products on int8 MFMA (gfx950).
//
// Computes the routed experts of src/diffuse-moe-graph.cpp:264-269 (ggml's
// mul_mat_id over Q4_K weights with Q8_K activations) and the shared expert of
// :280-286 (F32 activations, here two int8 digits), as one persistent launch
// per phase:
//   phase 0: h = silu(W_gate x) * (W_up x)       (gate and up of the same rows)
//   phase 1: y = W_down h
// (the conversion of h to the int8 layout runs in between, k_prep.hip).
//
// Arithmetic.  A Q4_K row is, per 256-value super-block, w = d*sc_j*q - dmin*m_j
// (j = 32-value sub-block, q in 0..15, sc_j, m_j 6-bit).  With int8
// activations a and their scale d_x this is ggml's vec_dot_q4_K_q8_K:
//   sum_k w a = d * sum_j sc_j S_j - dmin * sum_j m_j B_j,
//   S_j = sum_{k in j} q_k a_k (int32),  B_j = sum_{k in j} a_k.
// S_j comes from one v_mfma_i32_16x16x32_i8 per sub-block (the nibbles are the
// int8 operand), sum_j sc_j S_j from integer multiply-adds (exact), the min
// term from v_mfma_f32_16x16x16_f16 on the sums of 16 (exact integers in f16).
// The super-block result is scaled by d_x and accumulated in f32.
//
// Operand layout (checked on the hardware): srcA lane l = activation row l%16,
// k = 8*(l/16) + byte; srcB lane l = weight row l%16, same k; D lane l = weight
// row l%16, activation rows 4*(l/16)+i.  The tiled weight layout (k_quant.hip)
// puts the 32 quant bytes lane group g needs (bytes 32c + 8g .. +8 of each
// 32-byte chunk c: low nibbles = sub-block 2c, high = 2c+1) side by side, and
// repacks the 6-bit scales so that each is one bit-field extract.
//
// Memory.  A workgroup's four wavefronts share one work item: 16 activation
// rows, held whole (all K) in LDS for the item, so the wavefronts stream their
// weight tiles (coalesced 2304-byte runs) through a register ring with no
// workgroup barrier inside the item.
#include "dmoe_internal.h"

namespace dmoe {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Tuning constants (overridable at compile time).
#ifndef DMOE_X_STAGES
#define DMOE_X_STAGES 2          // register stages of the weight ring
#endif
#ifndef DMOE_X_DN_IT
#define DMOE_X_DN_IT 2           // row passes of a down item (shared activation tile)
#endif
#ifndef DMOE_X_BLOCKS
#define DMOE_X_BLOCKS 1024       // persistent grid
#endif
#ifndef DMOE_X_KC
#define DMOE_X_KC 2048           // activation values per row held in LDS at a time
#endif
#ifndef DMOE_X_WPE
#define DMOE_X_WPE 2             // wavefronts per SIMD the kernel is compiled for
#endif
constexpr int WAVES = 4;                     // waves per workgroup
constexpr int RT = 2;                        // 16-row weight tiles per wave per step
constexpr int STAGES = DMOE_X_STAGES;
constexpr int DN_IT = DMOE_X_DN_IT;
constexpr int GROWS_GU = WAVES * 16;             // gate/up rows of an item (gate and up tiles)
constexpr int GROWS_DN = WAVES * 16 * RT * DN_IT;   // down rows of an item
constexpr int TILE_BYTES = 16 * Q4K_BYTES;   // one tile x one super-block
constexpr int KC = DMOE_X_KC;

__device__ __forceinline__ float h16f(uint32_t u) { return (float)__builtin_bit_cast(_Float16, (uint16_t)u); }

struct Q4KTile {        // a lane's share of one 16-row tile in one super-block
    uint4 h;            // d, dmin, repacked scales
    uint4 q0, q1;       // the 32 quant bytes of lane group g
};

__device__ __forceinline__ void load_tile(Q4KTile &t, const uint8_t *tile, int sb, int r16, int g)
{
    const uint8_t *blk = tile + (size_t)sb * TILE_BYTES + r16 * Q4K_BYTES;
    t.h = *reinterpret_cast<const uint4 *>(blk);
    const uint4 *qp = reinterpret_cast<const uint4 *>(blk + 16 + 32 * g);
    t.q0 = qp[0];
    t.q1 = qp[1];
}

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t w)
{
    return __builtin_amdgcn_ubfe(v, off, w);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// The item's activation rows in LDS (dynamic shared memory):
//   q  [16][K + 16] int8   (row padding spreads the rows over the banks)
//   bs [16][K/16 + 8] f16
//   d  [nsb][16] f32
struct ATileView {
    int8_t *q;
    uint16_t *bs;
    float *d;
    int qs, bss;        // row strides (bytes, f16 elements)
};

__device__ __forceinline__ ATileView atile_view(uint8_t *lds, int K)
{
    ATileView v;
    v.qs = K + 16;
    v.bss = K / 16 + 8;
    v.q = reinterpret_cast<int8_t *>(lds);
    v.bs = reinterpret_cast<uint16_t *>(lds + 16 * v.qs);
    v.d = reinterpret_cast<float *>(lds + 16 * v.qs + 16 * v.bss * 2);
    return v;
}

size_t atile_bytes(int K)
{
    return (size_t)16 * (K + 16) + (size_t)16 * (K / 16 + 8) * 2 + (size_t)(K / 256) * 16 * 4;
}

// Copies values [k0, k0 + kc) of the item's 16 activation rows (global row
// rows[j], j < 16, in LDS) into the LDS tile; loads go out in rounds of eight
// 16-byte pieces per thread.
__device__ __forceinline__ void load_atile(const ActI8 &act, const int *rows, const ATileView &at,
                                           int k0, int kc, int tid)
{
    constexpr int T = WAVES * 64;
    const int K = act.K, nsb = K / 256;
    const int per_row = kc / 16;                 // 16-byte pieces of a q row
    const int nq = 16 * per_row;
    for (int base = 0; base < nq; base += 8 * T) {
        uint4 v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = min(base + i * T + tid, nq - 1);
            const int r = c / per_row, col = c - r * per_row;
            v[i] = *reinterpret_cast<const uint4 *>(act.q + (size_t)rows[r] * K + k0 + col * 16);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = base + i * T + tid;
            if (c < nq) {
                const int r = c / per_row, col = c - r * per_row;
                *reinterpret_cast<uint4 *>(at.q + r * at.qs + col * 16) = v[i];
            }
        }
    }
    const int bs_pieces = kc / 128;              // 16-byte pieces of a bs row
    for (int c = tid; c < 16 * bs_pieces; c += T) {
        const int r = c / bs_pieces, col = c - r * bs_pieces;
        const uint4 v = *reinterpret_cast<const uint4 *>(act.bs + (size_t)rows[r] * (K / 16) + k0 / 16 + col * 8);
        *reinterpret_cast<uint4 *>(at.bs + r * at.bss + col * 8) = v;
    }
    const int nsbc = kc / 256, sb0 = k0 / 256;
    for (int c = tid; c < 16 * nsbc; c += T) {
        const int r = c / nsbc, sb = c - r * nsbc;
        at.d[sb * 16 + r] = act.d[(size_t)rows[r] * nsb + sb0 + sb];
    }
}

// One super-block of RT weight tiles against the activation tile.
__device__ __forceinline__ void compute_sb(const Q4KTile (&cur)[RT], const ATileView &at, int sb,
                                           int r16, int g, float (&acc)[RT][4])
{
    // activation operands of the 8 sub-blocks: row r16, bytes 64g .. 64g+63
    const uint4 *ap = reinterpret_cast<const uint4 *>(at.q + r16 * at.qs + sb * 256 + 64 * g);
    const uint4 a01 = ap[0], a23 = ap[1], a45 = ap[2], a67 = ap[3];
    const long a[8] = {
        (long)((uint64_t)a01.y << 32 | a01.x), (long)((uint64_t)a01.w << 32 | a01.z),
        (long)((uint64_t)a23.y << 32 | a23.x), (long)((uint64_t)a23.w << 32 | a23.z),
        (long)((uint64_t)a45.y << 32 | a45.x), (long)((uint64_t)a45.w << 32 | a45.z),
        (long)((uint64_t)a67.y << 32 | a67.x), (long)((uint64_t)a67.w << 32 | a67.z)};
    const h4 ab = __builtin_bit_cast(h4, *reinterpret_cast<const uint2 *>(at.bs + r16 * at.bss + sb * 16 + 4 * g));
    const float4 dxv = *reinterpret_cast<const float4 *>(at.d + sb * 16 + 4 * g);
    const float dx[4] = {dxv.x, dxv.y, dxv.z, dxv.w};
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const Q4KTile &t = cur[r];
        // six-bit scales (repacked: sc0..sc4 | sc5..sc7 m0 m1 | m2..m6, m7 in bits 30..31)
        const uint32_t sc[8] = {bfe(t.h.y, 0, 6),  bfe(t.h.y, 6, 6),  bfe(t.h.y, 12, 6),
                                bfe(t.h.y, 18, 6), bfe(t.h.y, 24, 6), bfe(t.h.z, 0, 6),
                                bfe(t.h.z, 6, 6),  bfe(t.h.z, 12, 6)};
        const uint32_t msrc = g == 0 ? t.h.z : t.h.w;
        const uint32_t moff = g == 0 ? 18u : 12u * (uint32_t)g - 12u;
        const uint32_t m7 = (t.h.y >> 30) | ((t.h.z >> 30) << 2) | ((t.h.w >> 30) << 4);
        const uint32_t ma = bfe(msrc, moff, 6);
        const uint32_t mb = g == 3 ? m7 : bfe(msrc, moff + 6, 6);
        const _Float16 fa = (_Float16)(float)ma, fb = (_Float16)(float)mb;
        const h4 bm = {fa, fa, fb, fb};
        // nibbles -> int8 operands: dwords 2c, 2c+1 hold chunk c of lane group g
        const uint32_t w[8] = {t.q0.x, t.q0.y, t.q0.z, t.q0.w, t.q1.x, t.q1.y, t.q1.z, t.q1.w};
        int isum[4] = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t l0 = w[2 * c] & 0x0F0F0F0Fu, l1 = w[2 * c + 1] & 0x0F0F0F0Fu;
            const uint32_t h0 = (w[2 * c] >> 4) & 0x0F0F0F0Fu, h1 = (w[2 * c + 1] >> 4) & 0x0F0F0F0Fu;
            const long blo = (long)((uint64_t)l1 << 32 | l0), bhi = (long)((uint64_t)h1 << 32 | h0);
            v4i s_lo = {0, 0, 0, 0}, s_hi = {0, 0, 0, 0};
            s_lo = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[2 * c], blo, s_lo, 0, 0, 0);
            s_hi = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[2 * c + 1], bhi, s_hi, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) isum[i] += (int)sc[2 * c] * s_lo[i] + (int)sc[2 * c + 1] * s_hi[i];
        }
        f4 s2 = {0.0f, 0.0f, 0.0f, 0.0f};
        s2 = __builtin_amdgcn_mfma_f32_16x16x16f16(ab, bm, s2, 0, 0, 0);
        const float d = h16f(t.h.x & 0xffffu), dmin = h16f(t.h.x >> 16);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[r][i] += dx[i] * (d * (float)isum[i] - dmin * s2[i]);
    }
}

// Work items of phase 0: routed (work-list entry ec, group of 64 rows), then
// shared (chunk of 8 tokens, group of 64 rows); phase 1 the same with groups of
// GROWS_DN rows.  A routed item's 16 activation rows are the pairs of its
// entry (one expert, up to 16 consecutive pairs of it); a shared item's are the
// a1 / a0 digit rows of its 8 tokens interleaved (t a1, t a0, ...), so that each
// lane's four outputs are (t, a1), (t, a0), (t+1, a1), (t+1, a0) and the two
// digits' products are summed in-lane.
template <int PHASE>
__global__ __launch_bounds__(WAVES * 64, DMOE_X_WPE) void k_expert_q4k(MoeJob job)
{
    constexpr bool DOWN = PHASE == 1;
    constexpr int IT = DOWN ? DN_IT : 1;             // row passes per item
    constexpr int GROWS = DOWN ? GROWS_DN : GROWS_GU;
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int s_rows[16];

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
    const int Kin = DOWN ? FF : H;                   // reduction length (SF == FF when shared)
    const int nsb = Kin / 256;
    const int steps = IT * nsb;
    const int kc = min(Kin, KC);                     // values per LDS chunk (Kin % kc == 0)
    const int nsbc = kc / 256;
    const ATileView at = atile_view(lds, kc);

    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        const bool shared = item >= routed_items;
        const int j = shared ? item - routed_items : item;
        const int rgn = shared ? rg_sh : rg;
        const int unit = j / rgn;                 // work-list entry or shared chunk
        const int rbase = (j - unit * rgn) * GROWS;
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
        // this wave's weight tiles of pass it: tb[it][r]
        const uint8_t *tb[IT][RT];
        if (!DOWN) {
            const WTensor &a = shared ? job.sg : job.eg;
            const WTensor &b = shared ? job.su : job.eu;
            const int t16 = (rbase + wave * 16) / 16;
            tb[0][0] = a.data + (size_t)e * a.nb2 + (size_t)t16 * nsb * TILE_BYTES;
            tb[0][1] = b.data + (size_t)e * b.nb2 + (size_t)t16 * nsb * TILE_BYTES;
        } else {
            const WTensor &a = shared ? job.sd : job.ed;
#pragma unroll
            for (int it = 0; it < IT; it++)
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    const int t16 = (rbase + it * (WAVES * 32) + wave * 32) / 16 + r;
                    tb[it][r] = a.data + (size_t)e * a.nb2 + (size_t)t16 * nsb * TILE_BYTES;
                }
        }
        auto load_step = [&](Q4KTile (&t)[RT], int s) {
            const int sc = min(s, steps - 1);
            const int it = sc / nsb, sb = sc - it * nsb;
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const uint8_t *p = tb[0][r];
#pragma unroll
                for (int q = 1; q < IT; q++)
                    if (it == q) p = tb[q][r];
                load_tile(t[r], p, sb, r16, g);
            }
        };

        // weights of the first steps in flight while the activation tile loads
        Q4KTile ring[STAGES][RT];
#pragma unroll
        for (int st = 0; st < STAGES; st++) load_step(ring[st], st);
        const ActI8 &act = DOWN ? (shared ? job.ahs : job.ah) : (shared ? job.axs : job.ax);
        __syncthreads();                          // the previous item's LDS reads are done
        // activation row of item row jr: tokens in phase 0, pairs in phase 1;
        // shared rows interleave the a1 and a0 digit rows (a0 rows start at N)
        if (tid < 16) {
            int row;
            if (shared) {
                row = t_first + min(tid >> 1, nt - 1) + (tid & 1) * N;
            } else {
                const int p = job.perm[t_first + min(tid, nt - 1)];
                row = DOWN ? p : p / K;
            }
            s_rows[tid] = row;
        }
        __syncthreads();
        load_atile(act, s_rows, at, 0, kc, tid);
        __syncthreads();
        int chunk = 0;                            // K chunk in LDS

        float acc[IT][RT][4];
#pragma unroll
        for (int it = 0; it < IT; it++)
#pragma unroll
            for (int r = 0; r < RT; r++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[it][r][i] = 0.0f;
        // weight ring: compute step s from its stage, then refill that stage
        // with step s + STAGES (clamped: every step issues the same loads)
        for (int s0 = 0; s0 < steps; s0 += STAGES) {
#pragma unroll
            for (int st = 0; st < STAGES; st++) {
                const int s = s0 + st;
                if (s < steps) {
                    const int it = s / nsb, sb = s - it * nsb;
                    const int ck = sb / nsbc;
                    if (ck != chunk) {
                        // next K chunk of the activation rows (the weights stay in flight)
                        __syncthreads();
                        load_atile(act, s_rows, at, ck * kc, kc, tid);
                        __syncthreads();
                        chunk = ck;
                    }
#pragma unroll
                    for (int q = 0; q < IT; q++)
                        if (it == q) compute_sb(ring[st], at, sb - ck * nsbc, r16, g, acc[q]);
                }
                load_step(ring[st], s + STAGES);
            }
        }

        // results
        float *out = DOWN ? (shared ? job.ys : job.ye) : (shared ? job.hs : job.h);
        const int orows = DOWN ? H : (shared ? SF : FF);
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int row0 = DOWN ? rbase + it * (WAVES * 32) + wave * 32 : rbase + wave * 16;
            if (!shared) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (4 * g + i >= nt) continue;
                    float *o = out + (size_t)job.perm[t_first + 4 * g + i] * orows + row0 + r16;
                    if (!DOWN) {
                        o[0] = silu(acc[it][0][i]) * acc[it][1][i];
                    } else {
#pragma unroll
                        for (int r = 0; r < RT; r++) o[16 * r] = acc[it][r][i];
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i += 2) {
                    if (2 * g + (i >> 1) >= nt) continue;
                    float *o = out + (size_t)(t_first + 2 * g + (i >> 1)) * orows + row0 + r16;
                    if (!DOWN) {
                        o[0] = silu(acc[it][0][i] + acc[it][0][i + 1]) *
                               (acc[it][1][i] + acc[it][1][i + 1]);
                    } else {
#pragma unroll
                        for (int r = 0; r < RT; r++) o[16 * r] = acc[it][r][i] + acc[it][r][i + 1];
                    }
                }
            }
        }
    }
}

int expert_rows_per_item(int phase) { return phase == 0 ? GROWS_GU : GROWS_DN; }

bool expert_k_ok(int K) { return K % 256 == 0 && (K <= KC || K % KC == 0); }

hipError_t launch_expert_q4k(int phase, const MoeJob &job, hipStream_t s)
{
    if (job.FF % GROWS_GU || job.FF % 256 || job.H % GROWS_DN || job.H % 256 ||
        job.ax.K != job.H || job.ah.K != job.FF ||
        (job.has_shared && (job.SF != job.FF || job.ahs.K != job.SF)))
        return hipErrorInvalidValue;
    const int Kin = phase == 0 ? job.H : job.FF;
    if (Kin > KC && Kin % KC) return hipErrorInvalidValue;
    const size_t lds = atile_bytes(Kin < KC ? Kin : KC);
    static bool attr[2] = {false, false};
    if (!attr[phase]) {
        const void *k = phase == 0 ? (const void *)k_expert_q4k<0> : (const void *)k_expert_q4k<1>;
        const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 156 * 1024);
        if (e != hipSuccess) return e;
        attr[phase] = true;
    }
    if (phase == 0)
        hipLaunchKernelGGL(k_expert_q4k<0>, dim3(DMOE_X_BLOCKS), dim3(WAVES * 64), lds, s, job);
    else
        hipLaunchKernelGGL(k_expert_q4k<1>, dim3(DMOE_X_BLOCKS), dim3(WAVES * 64), lds, s, job);
    return hipGetLastError();
}

} // namespace dmoe

