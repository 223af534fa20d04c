// k_down_span.hip — down products of the Q4_K experts for few tokens, by
// spans of (unit, 16-row tile) work: src/diffuse-moe-graph.cpp:269 (down of
// every routed pair) and :285 (the shared expert's down); the weighted combine
// (:270-278, :286) is k_combine4's launch after it.
//
// Work division.  A unit is one work-list entry (one expert, up to 16 of its
// pairs) or one chunk of 8 tokens of the shared expert (their a1 / a0 digit
// rows, interleaved), as in k_down_rows.hip.  The launch's work is the list
// of (unit, tile) pairs in unit-major order, nu x (H / 16) of them, each four
// super-block steps at moe_ff 1024; workgroup b takes the contiguous range
// b W / G .. (b + 1) W / G - 1 of the W, and wavefront w of it the w-th
// eighth.  A range of at most 2 H / 16 tiles covers at most three units, whose
// activation rows (16 rows x moe_ff int8, sums of 16 and scales) are loaded
// into LDS once at the start: every activation byte is read once per
// workgroup that needs it, and each workgroup streams the same number of
// weight bytes.  (k_down_rows gives each workgroup 16 rows of every unit
// instead, which reads every unit's activation rows in every workgroup: two
// activation bytes per weight byte.)
//
// Weights go straight to registers, a ring of DS_R sets per wavefront loaded
// DS_R - 1 steps ahead (the compiler's own loads, so it counts their waits);
// the activations are in LDS, so the step loop has no barrier.  (Deeper
// rings measured slower: 26.8, 26.8, 27.0, 27.7, 28.5, 30.0, 31.8 us for 2,
// 3, 4, 5, 6, 8, 12 sets at 32 tokens; so did 16 wavefronts and two
// workgroups per CU.)  Each step's arithmetic is compute_sb's for one
// tile (k_expert.hip) with no fused multiply-adds, as k_down_rows computes
// it, so the products equal that kernel's bit for bit; they go to ye [pair][H] and ys [token][H] (the shared expert's
// two digits summed in-lane) for the combine launch.  Contraction is off for
// the whole file, the shared tile arithmetic included, as in k_down_rows.hip.
#pragma clang fp contract(off)
#include "dmoe_q4k.h"

#include <type_traits>

namespace dmoe {

constexpr int DS_WAVES = 8;
constexpr int DS_R = 3;            // weight register sets per wavefront (2 steps in flight)
constexpr int DS_SLOTS = 3;        // units whose activations a workgroup holds
constexpr int DS_MAX_SB = 4;       // super-blocks of the reduction (moe_ff <= 1024)
constexpr int DS_TAB_E = 1024;   // routed experts whose offsets and counts are staged in LDS
constexpr int DS_TAB_EC = 2048;  // work-list entries staged in LDS
constexpr int DS_TAB_P = 2048;   // (token, slot) pairs whose permutation entries are staged

typedef unsigned int ds_u4v __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) ds_u4v *ds_gu4v_ptr;

// f(integral_constant<int, J>) for J = J0 .. J1 - 1, as straight-line code
// (the register sets it indexes stay registers)
template <int J0, int J1, class F>
__device__ __forceinline__ void ds_unroll(F &&f)
{
    if constexpr (J0 < J1) {
        f(std::integral_constant<int, J0>());
        ds_unroll<J0 + 1, J1>(f);
    }
}

// 16-byte non-temporal load from global memory (the weights stream once)
__device__ __forceinline__ uint4 ds_ld_nt16(const void *p)
{
    const ds_u4v v = __builtin_nontemporal_load((ds_gu4v_ptr)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// TABS: the work list and the routing's offsets, counts and permutation fit
// the LDS tables (ds_tabs); they are loaded there at the start, all at once,
// and every lookup of the prologue after that is an LDS read.
template <bool TABS>
__global__ __launch_bounds__(DS_WAVES * 64) void k_down_span(DownRowsJob job)
{
#pragma clang fp contract(off)
    __shared__ __align__(16) uint8_t s_act[DS_SLOTS][DS_MAX_SB][ASTEP_BYTES];
    __shared__ const uint8_t *s_uw[DS_SLOTS];     // unit's weight matrix (tiled)
    __shared__ int32_t s_up0[DS_SLOTS];           // first pair (routed) / first token (shared)
    __shared__ int32_t s_unp[DS_SLOTS];           // pairs (> 0) / -tokens (shared)
    __shared__ int32_t s_pid[DS_SLOTS][16];       // routed: the unit's pair ids
    __shared__ int32_t s_ecx[TABS ? DS_TAB_EC : 1], s_ecc[TABS ? DS_TAB_EC : 1];
    __shared__ int32_t s_off[TABS ? DS_TAB_E : 1], s_cnt[TABS ? DS_TAB_E : 1], s_perm[TABS ? DS_TAB_P : 1];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int N = job.N, H = job.H, FF = job.FF;
    const int nsb = FF / 256, NT = H / 16;
    const int n_ec = job.wl.n_ec[0];
    // the work list and the routing tables, independent loads issued
    // together: one round trip, where the count, the entries, the offsets
    // and the pair ids in turn take four
    if constexpr (TABS) {
        for (int i = tid; i < job.ec_cap; i += DS_WAVES * 64) {
            s_ecx[i] = job.wl.ec_expert[i];
            s_ecc[i] = job.wl.ec_chunk[i];
        }
        for (int i = tid; i < job.E; i += DS_WAVES * 64) {
            s_off[i] = job.offsets[i];
            s_cnt[i] = job.counts[i];
        }
        for (int i = tid; i < N * job.K; i += DS_WAVES * 64) s_perm[i] = job.perm[i];
        __syncthreads();
    }
    const int nsh = job.has_shared ? (N + 7) / 8 : 0;
    const int nu = n_ec + nsh;
    const long W = (long)nu * NT;
    const long lo = W * blockIdx.x / gridDim.x, hi = W * (blockIdx.x + 1) / gridDim.x;
    if (lo >= hi) return;                          // the whole workgroup: no work
    const int u_first = (int)(lo / NT);
    const int nslot = min(DS_SLOTS, (int)((hi - 1) / NT) - u_first + 1);

    // the units' descriptors, then their pair ids
    if (tid < nslot) {
        const int u = u_first + tid;
        if (u < n_ec) {
            int e, c, off, cnt;
            if constexpr (TABS) {
                e = s_ecx[u];
                c = s_ecc[u];
                off = s_off[e];
                cnt = s_cnt[e];
            } else {
                e = job.wl.ec_expert[u];
                c = job.wl.ec_chunk[u];
                off = job.offsets[e];
                cnt = job.counts[e];
            }
            s_uw[tid] = job.ed.data + (size_t)e * job.ed.nb2;
            s_up0[tid] = off + EXPERT_CHUNK * c;
            s_unp[tid] = min(EXPERT_CHUNK, cnt - EXPERT_CHUNK * c);
        } else {
            const int c = u - n_ec;
            s_uw[tid] = job.sd.data;
            s_up0[tid] = 8 * c;
            s_unp[tid] = -min(8, N - 8 * c);
        }
    }
    __syncthreads();

    // this wavefront's tile-units i0 .. i1 - 1, nsb steps each: eighth
    // 2 (w % 4) + w / 4, so that the two wavefronts of one SIMD (w and
    // w + 4) take adjacent eighths, which together hold a quarter of the
    // range to within one tile (eighths alternate between the floor and the
    // ceiling of a fractional size)
    const long L = hi - lo;
    const int e8 = 2 * (wave & 3) + (wave >> 2);
    const long i0 = lo + L * e8 / DS_WAVES, i1 = lo + L * (e8 + 1) / DS_WAVES;
    const int Q = (int)(i1 - i0) * nsb;
    // a step's place: unit slot, tile, super-block
    struct Cur {
        int sl, t, sb;
    };
    auto start = [&](Cur &c) {
        const int u = (int)(i0 / NT);
        c.sl = u - u_first;
        c.t = (int)(i0 - (long)u * NT);
        c.sb = 0;
    };
    auto advance = [&](Cur &c) {
        if (++c.sb == nsb) {
            c.sb = 0;
            if (++c.t == NT) {
                c.t = 0;
                c.sl++;
            }
        }
    };
    // the load cursor runs DS_R - 1 steps ahead and stays on the last step
    // (loading it again, never used) once it gets there
    Cur lc, cc;
    start(lc);
    start(cc);
    int lq = 0;
    auto load = [&](Q4KTile &o) {
        const uint4 *wp = reinterpret_cast<const uint4 *>(s_uw[min(lc.sl, DS_SLOTS - 1)] +
                                                          ((size_t)lc.t * nsb + lc.sb) * TILE_BYTES);
        o.h = ds_ld_nt16(wp + r16);
        o.q0 = ds_ld_nt16(wp + (1 + 2 * g) * 16 + r16);
        o.q1 = ds_ld_nt16(wp + (2 + 2 * g) * 16 + r16);
        if (lq + 1 < Q) {
            lq++;
            advance(lc);
        }
    };
    float acc[1][4] = {{0.0f, 0.0f, 0.0f, 0.0f}};
    auto compute = [&](const Q4KTile &w) {
        const int sl = min(cc.sl, DS_SLOTS - 1);
        const Q4KTile cur[1] = {w};
        compute_sb<1>(cur, &s_act[sl][cc.sb][0], r16, g, acc);
        if (cc.sb == nsb - 1) {
            // products of (unit, tile t): rows 16 t + r16, block rows 4 g + i
            const int np = s_unp[sl], row = 16 * cc.t + r16;
            if (np > 0) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (4 * g + i < np) job.ye[(size_t)s_pid[sl][4 * g + i] * H + row] = acc[0][i];
            } else {
#pragma unroll
                for (int i = 0; i < 4; i += 2) {
                    const int q2 = 2 * g + (i >> 1);
                    if (q2 < -np) job.ys[(size_t)(s_up0[sl] + q2) * H + row] = acc[0][i] + acc[0][i + 1];
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) acc[0][i] = 0.0f;
        }
        advance(cc);
    };
    // DS_R register sets: step s computes set s % DS_R, whose loads were
    // issued DS_R - 1 steps before; the set freed by step s - 1 takes step
    // s + DS_R - 1's loads first.  The first DS_R - 1 steps' weights need
    // only the units' matrices: they are issued before the pair ids and
    // activation rows are looked up.
    Q4KTile o[DS_R];
    if (Q > 0) ds_unroll<0, DS_R - 1>([&](auto jc) { load(o[decltype(jc)::value]); });
    if (tid < 16 * nslot) {
        const int sl = tid >> 4, i = tid & 15, np = s_unp[sl];
        if (np > 0) {
            const int pi = s_up0[sl] + min(i, np - 1);
            if constexpr (TABS)
                s_pid[sl][i] = s_perm[pi];
            else
                s_pid[sl][i] = job.perm[pi];
        }
    }
    __syncthreads();

    // Activation rows of every slot and super-block (k_expert.hip's loads of
    // one step: wavefronts 0..3 the q rows, 4 the sums of 16, 5 the scales;
    // block row ar of a unit: its pair (routed, the last repeated past the
    // unit's pairs) or token t's digit ar % 2 (shared))
    const int ar = wave < 4 ? 4 * wave + (lane >> 4) : (wave == 4 ? (lane >> 1) & 15 : lane & 15);
    const int aunit = (lane & 15) ^ (ar & 11);
    const bool aload = wave < 4 || (wave == 4 && lane < 32) || (wave == 5 && lane < 16);
    if (wave < ADMA_WAVES) {
        for (int sl = 0; sl < nslot; sl++) {
            const int np = s_unp[sl];
            const bool routed = np > 0;
            const ActI8 &act = routed ? job.ah : job.ahs;
            const int arow = routed ? s_pid[sl][ar] : s_up0[sl] + min(ar >> 1, -np - 1) + (ar & 1) * N;
            for (int sb = 0; sb < nsb; sb++) {
                uint8_t *st = &s_act[sl][sb][0];
                if (wave < 4)
                    lds_load16(act.q + (size_t)arow * FF + sb * 256 + aunit * 16, st + 1024 * wave);
                else if (wave == 4 && aload)
                    lds_load16(act.bs + (size_t)arow * (FF / 16) + sb * 16 + (lane & 1) * 8, st + ABS_OFF);
                else if (wave == 5 && aload)
                    lds_load4(act.d + (size_t)arow * nsb + sb, st + AD_OFF);
            }
        }
    }

    // The activation loads (and the weight loads issued before them) have
    // landed in every wavefront; the compiler, which does not see the
    // activation loads, counts its own weight loads' waits as issued.
    EXPERT_WAIT_VM(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    if (Q == 0) return;
    // whole rounds of DS_R steps without a test per step (so the waits the
    // compiler counts stay exact), then the last steps
    int s0 = 0;
    for (; s0 + DS_R <= Q; s0 += DS_R)
        ds_unroll<0, DS_R>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            load(o[(j + DS_R - 1) % DS_R]);
            compute(o[j]);
        });
    ds_unroll<0, DS_R - 1>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if (s0 + j < Q) {
            load(o[(j + DS_R - 1) % DS_R]);
            compute(o[j]);
        }
    });
}

// A workgroup's range must cover at most DS_SLOTS units: at most
// (DS_SLOTS - 1) H / 16 tile-units for the longest work list (ec_cap entries).
static bool span_fits(int N, int H, int ec_cap, int has_shared, int n_cu)
{
    const long NT = H / 16;
    const long nu_max = (long)ec_cap + (has_shared ? (N + 7) / 8 : 0);
    return n_cu > 0 && (nu_max * NT + n_cu - 1) / n_cu <= (DS_SLOTS - 1) * NT;
}

bool down_span_ok(int N, int K, int E, int H, int FF, int has_shared)
{
    int n_cu = 0;
    if (N <= 0 || K <= 0 || H % 16 || FF % 256 || FF / 256 > DS_MAX_SB || device_cu_count(&n_cu) != hipSuccess)
        return false;
    return span_fits(N, H, E + N * K / EXPERT_CHUNK + 1, has_shared, n_cu);
}

hipError_t launch_down_span(const DownRowsJob &job, hipStream_t s)
{
    int n_cu = 0;
    const hipError_t e = device_cu_count(&n_cu);
    if (e != hipSuccess) return e;
    if (!down_span_ok(job.N, job.K, job.E, job.H, job.FF, job.has_shared) ||
        !span_fits(job.N, job.H, job.ec_cap, job.has_shared, n_cu) ||
        job.wl.chunk != EXPERT_CHUNK || job.ah.K != job.FF || (job.has_shared && job.ahs.K != job.FF) ||
        !job.ye || (job.has_shared && !job.ys))
        return hipErrorInvalidValue;
    if (job.E <= DS_TAB_E && job.ec_cap <= DS_TAB_EC && job.N * job.K <= DS_TAB_P)
        hipLaunchKernelGGL(k_down_span<true>, dim3(n_cu), dim3(DS_WAVES * 64), 0, s, job);
    else
        hipLaunchKernelGGL(k_down_span<false>, dim3(n_cu), dim3(DS_WAVES * 64), 0, s, job);
    return hipGetLastError();
}

} // namespace dmoe
