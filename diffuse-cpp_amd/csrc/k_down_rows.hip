// k_down_rows.hip — down products of the Q4_K experts and the weighted
// combine in one launch, for few tokens (at most DR_MAX_PAIRS (token, slot)
// pairs): src/diffuse-moe-graph.cpp:269 (down of every routed pair), :270-278
// (weighted left fold over the slots) and :285-286 (shared expert's down,
// added last).
//
// Work division.  Workgroup b owns output rows 16 b .. 16 b + 15 of every
// expert: it streams the 16-row tile of each touched expert's down matrix
// (and of the shared expert's), so H / 16 workgroups read disjoint weight
// bytes and each reads the same amount (one per compute unit at H = 4096).
// A unit of work is one work-list entry (one expert, up to 16 of its pairs)
// or one chunk of 8 tokens of the shared expert (their a1 / a0 digit rows,
// interleaved); wavefront w takes units w, w + 8, ...  Each unit is K/256
// steps of one super-block.
//
// Operands go straight to registers: a lane loads its share of the weight
// tile (three 16-byte pieces of the tiled layout, non-temporal) and its
// activation operands (row r16's 64 bytes of lane group g, its sums of 16 and
// its scale; a lane's four output columns take theirs from lanes 4g .. 4g + 3
// by ds_bpermute) four steps ahead of their use; the
// step loop is unrolled five ways so that no register copy waits on a load.
// The arithmetic of a step is that of the Q4_K expert kernel (k_expert.hip),
// in the same order, so the products equal that kernel's bit for bit.
//
// Results stay in LDS ([pair][16] and [token][16] f32); after a barrier each
// output (token, row) is the left fold of its slots' products in slot order
// plus the shared expert's value, as k_combine computes it.
#include "dmoe_device.h"

namespace dmoe {

constexpr int DR_WAVES = 8;
constexpr int DR_AHEAD = 4;                      // steps in flight per wavefront
constexpr int DR_MAX_E = 1024;
constexpr int DR_MAX_UNITS = DR_MAX_E + DR_MAX_PAIRS / EXPERT_CHUNK + 1 + DR_MAX_TOKENS / 8;
constexpr int DR_TILE = 16 * Q4K_BYTES;          // 16 rows x one super-block (2304 bytes)
static_assert(EXPERT_CHUNK == 16, "one MFMA column block per work-list entry");

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4v __attribute__((ext_vector_type(4)));

typedef const __attribute__((address_space(1))) u4v *gu4v_ptr;

// 16-byte non-temporal load from global memory (a global, not flat, load: the
// pointer is read back from LDS, so its address space is stated here)
__device__ __forceinline__ uint4 ld_nt16(const void *p)
{
    const u4v v = __builtin_nontemporal_load((gu4v_ptr)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float dr_h16f(uint32_t u) { return (float)__builtin_bit_cast(_Float16, (uint16_t)u); }

// A lane's operands of one step.
struct DrOps {
    uint4 h, q0, q1;        // weight tile: d, dmin, repacked scales; quant bytes of lane group g
    uint4 a0, a1, a2, a3;   // activation row r16: the 8-byte operands of sub-blocks 0..7
    uint2 bs;               // its f16 sums of 16 (lane group g's four)
    float dself;            // scale of activation row r16 (rows 4g .. 4g + 3 are read from lanes 4g .. 4g + 3)
};

// One super-block of one 16-row tile against 16 activation rows: the
// arithmetic of compute_sb (k_expert.hip) for a single tile.
__device__ __forceinline__ void dr_compute(const DrOps &o, int g, float (&acc)[4])
{
#pragma clang fp contract(off)
    const long a[8] = {
        (long)((uint64_t)o.a0.y << 32 | o.a0.x), (long)((uint64_t)o.a0.w << 32 | o.a0.z),
        (long)((uint64_t)o.a1.y << 32 | o.a1.x), (long)((uint64_t)o.a1.w << 32 | o.a1.z),
        (long)((uint64_t)o.a2.y << 32 | o.a2.x), (long)((uint64_t)o.a2.w << 32 | o.a2.z),
        (long)((uint64_t)o.a3.y << 32 | o.a3.x), (long)((uint64_t)o.a3.w << 32 | o.a3.z)};
    const h4 ab = __builtin_bit_cast(h4, o.bs);
    const uint4 &t = o.h;
    const uint32_t sc[8] = {
        __builtin_amdgcn_ubfe(t.y, 0, 6),  __builtin_amdgcn_ubfe(t.y, 6, 6),
        __builtin_amdgcn_ubfe(t.y, 12, 6), __builtin_amdgcn_ubfe(t.y, 18, 6),
        __builtin_amdgcn_ubfe(t.y, 24, 6), __builtin_amdgcn_ubfe(t.z, 0, 6),
        __builtin_amdgcn_ubfe(t.z, 6, 6),  __builtin_amdgcn_ubfe(t.z, 12, 6)};
    const uint32_t msrc = g == 0 ? t.z : t.w;
    const uint32_t moff = g == 0 ? 18u : 12u * (uint32_t)g - 12u;
    const uint32_t m7 = (t.y >> 30) | ((t.z >> 30) << 2) | ((t.w >> 30) << 4);
    const uint32_t ma = __builtin_amdgcn_ubfe(msrc, moff, 6);
    const uint32_t mb = g == 3 ? m7 : __builtin_amdgcn_ubfe(msrc, moff + 6, 6);
    const _Float16 fa = (_Float16)(float)ma, fb = (_Float16)(float)mb;
    const h4 bm = {fa, fa, fb, fb};
    const uint32_t w[8] = {o.q0.x, o.q0.y, o.q0.z, o.q0.w, o.q1.x, o.q1.y, o.q1.z, o.q1.w};
    v4i sj[8];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t l0 = w[2 * c] & 0x0F0F0F0Fu, l1 = w[2 * c + 1] & 0x0F0F0F0Fu;
        const uint32_t h0 = (w[2 * c] >> 4) & 0x0F0F0F0Fu, h1 = (w[2 * c + 1] >> 4) & 0x0F0F0F0Fu;
        const long blo = (long)((uint64_t)l1 << 32 | l0), bhi = (long)((uint64_t)h1 << 32 | h0);
        const v4i z = {0, 0, 0, 0};
        sj[2 * c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[2 * c], blo, z, 0, 0, 0);
        sj[2 * c + 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[2 * c + 1], bhi, z, 0, 0, 0);
    }
    int isum[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            isum[i] = __mul24((int)sc[j], sj[j][i]) + isum[i];
            asm volatile("" : "+v"(isum[i]));
        }
    f4 s2 = {0.0f, 0.0f, 0.0f, 0.0f};
    s2 = __builtin_amdgcn_mfma_f32_16x16x16f16(ab, bm, s2, 0, 0, 0);
    const float d = dr_h16f(t.x & 0xffffu), dmin = dr_h16f(t.x >> 16);
    // scales of this lane's output columns: rows 4g + i, held by lanes 4g + i
    float dx[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        dx[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((4 * g + i) << 2,
                                                                       __builtin_bit_cast(int, o.dself)));
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = q4k_epi(acc[i], dx[i], d, (float)isum[i], dmin, s2[i]);
}

__global__ __launch_bounds__(DR_WAVES * 64) void k_down_rows(DownRowsJob job)
{
#pragma clang fp contract(off)
    __shared__ float y_s[DR_MAX_PAIRS * 16];          // routed products [pair id][row]
    __shared__ float ys_s[DR_MAX_TOKENS * 16];        // shared expert [token][row]
    __shared__ int32_t s_perm[DR_MAX_PAIRS];
    __shared__ int32_t s_off[DR_MAX_E], s_cnt[DR_MAX_E];
    __shared__ const uint8_t *s_uw[DR_MAX_UNITS];     // unit's weight tile (super-block 0)
    __shared__ int32_t s_up0[DR_MAX_UNITS];           // first pair (routed) / first token (shared)
    __shared__ int32_t s_unp[DR_MAX_UNITS];           // pairs (> 0) / -tokens (shared)

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int N = job.N, K = job.K, P = N * K, E = job.E, H = job.H, FF = job.FF;
    const int nsb = FF / 256;
    const size_t tile_off = (size_t)blockIdx.x * nsb * DR_TILE;

    // One round of independent loads: permutation, offsets, counts and the
    // work list (up to its allocated length) into LDS.
    const int n_ec = job.wl.n_ec[0];
    for (int i = tid; i < P; i += DR_WAVES * 64) s_perm[i] = job.perm[i];
    for (int i = tid; i < E; i += DR_WAVES * 64) {
        s_off[i] = job.offsets[i];
        s_cnt[i] = job.counts[i];
    }
    for (int u = tid; u < job.ec_cap; u += DR_WAVES * 64) {
        s_up0[u] = job.wl.ec_expert[u];
        s_unp[u] = job.wl.ec_chunk[u];
    }
    __syncthreads();
    const int nsh = job.has_shared ? (N + 7) / 8 : 0;
    const int nu = n_ec + nsh;
    for (int u = tid; u < nu; u += DR_WAVES * 64) {
        if (u < n_ec) {
            const int e = s_up0[u], c = s_unp[u];
            s_uw[u] = job.ed.data + (size_t)e * job.ed.nb2 + tile_off;
            s_up0[u] = s_off[e] + EXPERT_CHUNK * c;
            s_unp[u] = min(EXPERT_CHUNK, s_cnt[e] - EXPERT_CHUNK * c);
        } else {
            const int c = u - n_ec;
            s_uw[u] = job.sd.data + tile_off;
            s_up0[u] = 8 * c;
            s_unp[u] = -min(8, N - 8 * c);
        }
    }
    __syncthreads();

    // A projection (K == 0: shared units only, at most N / 8 of them, fewer
    // than the wavefronts) splits the units' super-blocks instead: wavefront w
    // takes the contiguous range of (unit, super-block) steps w T / 8 ..
    // (w + 1) T / 8 - 1 of the T = units x nsb, and leaves the partial sums of
    // the units it touches in its own slot of LDS (aliasing the routed
    // products, unused here), added in wavefront order after the barrier.
    const bool ksplit = K == 0;
    float *ps = y_s;                                   // [DR_WAVES][N][16] partial sums
    if (ksplit) {
        for (int i = tid; i < DR_WAVES * N * 16; i += DR_WAVES * 64) ps[i] = 0.0f;
        __syncthreads();
    }
    // Activation row of row j of a unit (rows past the unit's last repeat
    // it), without branches: every load of a step is issued unconditionally,
    // so the vector-memory counter waits stay exact across the step loop.
    auto act_row = [&](int np, int p0, int j) -> int {
        const bool routed = np > 0;
        const int pr = s_perm[p0 + (routed ? min(j, np - 1) : 0)];
        return routed ? pr : p0 + min(j >> 1, -np - 1) + (j & 1) * N;
    };
    // The load cursor's unit: its addresses are resolved once per unit (the
    // weight tile base is wave-uniform, the activation bases are per lane)
    // and each step adds the super-block's offset.
    struct Cursor {
        const uint8_t *w;        // weight tile, super-block 0 (wave-uniform)
        const int8_t *aq;        // row r16's operand bytes of lane group g, super-block 0
        const uint16_t *abs;     // its sums of 16
        const float *ad;         // scale of row r16, super-block 0
    };
    auto resolve = [&](int u, Cursor &c) {
        const int np = s_unp[u], p0 = s_up0[u];
        const uint64_t wb = (uint64_t)(uintptr_t)s_uw[u];
        c.w = (const uint8_t *)(uintptr_t)((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)wb) |
                                           ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(wb >> 32)) << 32));
        const bool routed = np > 0;
        const int8_t *q = routed ? job.ah.q : job.ahs.q;
        const uint16_t *bsp = routed ? job.ah.bs : job.ahs.bs;
        const float *dp = routed ? job.ah.d : job.ahs.d;
        const int ra = act_row(np, p0, r16);
        c.aq = q + (size_t)ra * FF + 64 * g;
        c.abs = bsp + (size_t)ra * (FF / 16) + 4 * g;
        c.ad = dp + (size_t)ra * nsb;
    };
    auto load = [&](const Cursor &c, int sb, DrOps &o) {
        const uint4 *wp = reinterpret_cast<const uint4 *>(c.w + (size_t)sb * DR_TILE);
        o.h = ld_nt16(wp + r16);
        o.q0 = ld_nt16(wp + (1 + 2 * g) * 16 + r16);
        o.q1 = ld_nt16(wp + (2 + 2 * g) * 16 + r16);
        const uint4 *aq = reinterpret_cast<const uint4 *>(c.aq + sb * 256);
        o.a0 = aq[0];
        o.a1 = aq[1];
        o.a2 = aq[2];
        o.a3 = aq[3];
        o.bs = *reinterpret_cast<const uint2 *>(c.abs + sb * 16);
        o.dself = c.ad[sb];
    };
    auto store = [&](int u, const float (&acc)[4]) {
        const int np = s_unp[u], p0 = s_up0[u];
        if (ksplit) {
#pragma unroll
            for (int i = 0; i < 4; i += 2)
                if (2 * g + (i >> 1) < -np) ps[(wave * N + p0 + 2 * g + (i >> 1)) * 16 + r16] = acc[i] + acc[i + 1];
            return;
        }
        if (np > 0) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (4 * g + i < np) y_s[s_perm[p0 + 4 * g + i] * 16 + r16] = acc[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; i += 2)
                if (2 * g + (i >> 1) < -np) ys_s[(p0 + 2 * g + (i >> 1)) * 16 + r16] = acc[i] + acc[i + 1];
        }
    };

    // This wavefront's steps: units wave, wave + 8, ..., nsb steps each.
    // DR_AHEAD steps are in flight while one is computed: a step's operands
    // are loaded into the register set the previous step has just consumed,
    // before this step's arithmetic.  Every load is issued in consumption
    // order, so waiting for one step's operands never waits for a later
    // step's (the vector-memory counter completes in issue order).
    const int ustride = ksplit ? 1 : DR_WAVES;
    int S, u_first, sb_first;
    if (ksplit) {
        const int T = nu * nsb, t0 = wave * T / DR_WAVES, t1 = (wave + 1) * T / DR_WAVES;
        S = t1 - t0;
        u_first = S > 0 ? t0 / nsb : 0;
        sb_first = S > 0 ? t0 - u_first * nsb : 0;
    } else {
        const int nk = wave < nu ? (nu - 1 - wave) / DR_WAVES + 1 : 0;
        S = nk * nsb;
        u_first = wave;
        sb_first = 0;
    }
    if (S > 0) {
        int lu = u_first, lsb = sb_first, ls = 0;          // next step to load (clamped to the last)
        Cursor lc;
        resolve(lu, lc);
        auto next = [&]() {
            if (ls + 1 < S) {
                ls++;
                if (++lsb == nsb) {
                    lsb = 0;
                    lu += ustride;
                    resolve(lu, lc);
                }
            }
        };
        DrOps o0, o1, o2, o3, o4;
        static_assert(DR_AHEAD == 4, "five register sets below");
        load(lc, lsb, o0);
        next();
        load(lc, lsb, o1);
        next();
        load(lc, lsb, o2);
        next();
        load(lc, lsb, o3);
        next();
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        int cu = u_first, csb = sb_first, cs = 0;
        auto step = [&](DrOps &cur, DrOps &ahead) {
            load(lc, lsb, ahead);
            next();
            dr_compute(cur, g, acc);
            ++cs;
            if (++csb == nsb || cs == S) {
                // a unit's last super-block, or (split) the end of the range
                store(cu, acc);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = 0.0f;
                csb = 0;
                cu += ustride;
            }
        };
        for (int s = 0; s < S; s += 5) {
            step(o0, o4);
            if (s + 1 < S) step(o1, o0);
            if (s + 2 < S) step(o2, o1);
            if (s + 3 < S) step(o3, o2);
            if (s + 4 < S) step(o4, o3);
        }
    }
    __syncthreads();

    // combine: out[t][row] = ((y_0 w_0 + y_1 w_1) + ...) + y_shared; with no
    // routed pairs (K == 0: a plain projection through the shared slot) the
    // shared value alone
    float *out = job.y + (size_t)blockIdx.x * 16;
    for (int o = tid; o < N * 16; o += DR_WAVES * 64) {
        const int t = o >> 4, r = o & 15;
        float a;
        if (ksplit) {
            a = ps[t * 16 + r];
            for (int w = 1; w < DR_WAVES; w++) a = a + ps[(w * N + t) * 16 + r];
        } else if (K > 0) {
            const float *wt = job.weights + (size_t)t * K;
            a = y_s[(t * K) * 16 + r] * wt[0];
            for (int k = 1; k < K; k++) a = a + y_s[(t * K + k) * 16 + r] * wt[k];
            if (job.has_shared) a = a + ys_s[t * 16 + r];
        } else {
            a = ys_s[t * 16 + r];
        }
        out[(size_t)t * H + r] = a;
    }
}

bool down_rows_ok(int N, int K, int E, int H, int FF)
{
    return N > 0 && N <= DR_MAX_TOKENS && K >= 0 && N * K <= DR_MAX_PAIRS && E <= DR_MAX_E && H % 16 == 0 &&
           FF % 256 == 0;
}

hipError_t launch_down_rows(const DownRowsJob &job, hipStream_t s)
{
    if (!down_rows_ok(job.N, job.K, job.E, job.H, job.FF) ||
        job.ec_cap + (job.has_shared ? (job.N + 7) / 8 : 0) > DR_MAX_UNITS ||
        job.wl.chunk != EXPERT_CHUNK || (job.K > 0 && job.ah.K != job.FF) ||
        (job.has_shared && job.ahs.K != job.FF) || (job.K == 0 && (!job.has_shared || job.ec_cap != 0)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_down_rows, dim3(job.H / 16), dim3(DR_WAVES * 64), 0, s, job);
    return hipGetLastError();
}

} // namespace dmoe
