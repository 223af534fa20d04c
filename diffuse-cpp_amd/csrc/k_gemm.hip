// k_gemm.hip — grouped F16 expert products on MFMA (gfx950), the prefill path.
//
// Computes the routed experts of src/diffuse-moe-graph.cpp:264-269 for F16
// expert weights (ggml's mul_mat_id converts the activations to F16, its
// vec_dot_type, and accumulates f16 x f16 products in f32) and the shared
// expert of :280-286 (F32 semantics: its F16 weights are exact, the f32
// activations run as two f16 passes, hi = f16(x) and lo = f16(x - hi)):
//   phase 0: h = silu(W_gate x) * (W_up x), written as the f16 activations of
//            phase 1 (routed) or as their hi / lo pair (shared)
//   phase 1: y = W_down h
//
// Work item: one expert, a block of up to 256 of its (token, slot) pairs (or
// 256 tokens of the shared expert) and a group of output rows (128 moe_ff rows
// of gate and of up, or 256 n_embd rows of down).  Items of one expert and
// row group but different pair blocks are a row-group count apart, so they run
// together and share the weight rows through the caches.  Each 32-wide k
// step stages the 256 activation rows and the 256 weight rows in LDS with the
// LDS-direct global loads (global_load_lds_dwordx4: no registers held, so a
// 4-stage ring keeps three steps of loads in flight to cover HBM latency);
// each of the 8 wavefronts computes a 128 x 64 output
// tile as 8 x 4 v_mfma_f32_16x16x32_f16 (operand layout as in k_expert.hip: srcA lane l =
// activation row l%16, k = 8*(l/16)+e; srcB = weight row, same k; D lane l =
// weight row l%16, activation rows 4*(l/16)+i).
#include "dmoe_internal.h"

namespace dmoe {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int GWAVES = 8;
constexpr int GT = GWAVES * 64;      // threads per workgroup
constexpr int GNW = 256;             // weight rows per item (gate/up: 128 moe_ff rows of each)
constexpr int GS = 4;                // LDS pipeline stages
constexpr int GTILE = GM * GK * 2;   // bytes of one operand tile of a stage (64-byte rows)
constexpr int GP = GM * GK / 8 / GT; // 16-byte pieces per thread per tile and stage

__device__ __forceinline__ float gsilu(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ uint16_t f2h_rn(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// The 16-byte k-chunk q (0..3) of tile row r sits in slot q ^ swz(r) of the
// row.  A ds_read_b128 serves 16 lanes per cycle over the 64 banks: the four
// lane quads (4 consecutive lanes) of one half-wave whose quad indices have
// equal bit parity (measured on gfx950 with the LDS bank-conflict counter).
// The operand reads (lane l: row l % 16, chunk l / 16) are conflict-free
// with the slot flipped by row bits 1..2.
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 3; }

// s_waitcnt with vmcnt(n), lgkmcnt(0), expcnt untouched (n < 16)
#define GEMM_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(0x70 | (n))

// LDS-direct load of 16 bytes per lane: lane l's bytes go to LDS address
// lds + 16 l (lds wave-uniform).  Written as inline assembly so that the
// compiler does not order every later LDS read after it (it cannot tell the
// ring's buffers apart and would wait for all loads in flight); completion is
// awaited explicitly with GEMM_WAIT_VM before the barrier of each step.
__device__ __forceinline__ void lds_load16(const void *src, const void *lds)
{
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(m0) : "memory", "m0");
}

template <int PHASE>
__global__ __launch_bounds__(GT) void k_gemm_f16(GemmJob job)
{
    constexpr bool DOWN = PHASE == 1;
    constexpr int GN = DOWN ? GN_DN : GN_GU;         // output rows per item
    static_assert(GP * GT * 8 == GM * GK && GNW == GM && GP == 2, "tile shapes");
    // stage s: activation tile at S[s][0], weight tile at S[s][1]; row r of a
    // tile is 64 bytes at r * 64, its k-chunks swizzled by swz(r)
    __shared__ __align__(16) uint8_t S[GS][2][GTILE];
    __shared__ int s_arow[GM];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int N = job.n_tokens, K = job.top_k;
    const int H = job.H, FF = job.FF, SF = job.SF;
    const int n_ec = job.wl.n_ec[0];
    const int nch = job.has_shared ? (N + GM - 1) / GM : 0;
    const int rg = (DOWN ? H : FF) / GN, rg_sh = (DOWN ? H : SF) / GN;
    // Items by XCD: workgroup b runs on XCD b % 8 (round-robin dispatch).  The
    // units (expert chunks, expert-major, then the shared expert's token
    // chunks) are split into 8 contiguous segments of equal work (a shared
    // unit does two passes), one per XCD, so that the row groups of a unit
    // (one activation block) and the chunks of an expert (one weight slice)
    // meet in the same L2.  Within a segment, item m is unit m / row-groups,
    // row group m % row-groups.
    static_assert(GEMM_BLOCKS % 8 == 0, "grid by XCD");
    const int xcd = blockIdx.x & 7, G8 = gridDim.x >> 3, lb = blockIdx.x >> 3;
    const long w_routed = (long)n_ec * rg, w_total = w_routed + 2L * nch * rg_sh;
    auto seg = [&](int x) -> int {
        const long t = w_total * x / 8;
        return t <= w_routed ? (int)((t + rg - 1) / rg)
                             : n_ec + (int)((t - w_routed + 2 * rg_sh - 1) / (2 * rg_sh));
    };
    const int u0 = seg(xcd), u1 = seg(xcd + 1);
    const int nr = max(0, min(u1, n_ec) - u0);                             // routed units
    const int s0 = max(u0, n_ec) - n_ec, ns = max(0, u1 - max(u0, n_ec)); // shared chunks
    const int seg_items = nr * rg + ns * rg_sh;
    // wave grid 2 (activation rows) x 4 (weight rows): 128 x 64 per wave
    const int tok0 = 128 * (wave >> 2);
    const int wq = wave & 3;
    // weight rows of this wave's four 16-row tiles in the weight tile: gate/up:
    // 32 moe_ff rows of gate (tiles 0, 1) and the same rows of up (tiles 2, 3)
    int brow[4];
#pragma unroll
    for (int tw = 0; tw < 4; tw++)
        brow[tw] = DOWN ? 64 * wq + 16 * tw
                        : (tw < 2 ? 32 * wq + 16 * tw : GN + 32 * wq + 16 * (tw - 2));
    // byte offsets of this lane's operand chunk g in a tile
    int aoff[8], boff[4];
#pragma unroll
    for (int ti = 0; ti < 8; ti++) {
        const int r = tok0 + 16 * ti + r16;
        aoff[ti] = r * 64 + ((g ^ swz(r)) << 4);
    }
#pragma unroll
    for (int tw = 0; tw < 4; tw++) {
        const int r = brow[tw] + r16;
        boff[tw] = r * 64 + ((g ^ swz(r)) << 4);
    }

    for (int m = lb; m < seg_items; m += G8) {
        const bool shared = m >= nr * rg;
        const int mm = shared ? m - nr * rg : m;
        const int rgn = shared ? rg_sh : rg;
        const int unit = (shared ? s0 : u0) + mm / rgn, rb = mm % rgn;
        int t_first, nt, e = 0;
        if (!shared) {
            e = job.wl.ec_expert[unit];
            const int c0 = job.wl.ec_chunk[unit] * GM;
            t_first = job.offsets[e] + c0;
            nt = min(GM, job.counts[e] - c0);
        } else {
            t_first = unit * GM;
            nt = min(GM, N - t_first);
        }
        const int Kin = DOWN ? (shared ? SF : FF) : H;
        const int nsteps = Kin / GK;
        const int total_steps = (shared ? 2 : 1) * nsteps;
        // activations: rows of a [rows][Kin] f16 array (split: lo rows after the hi rows)
        const uint16_t *A = DOWN ? (shared ? job.hs16 : job.h16) : (shared ? job.xs16 : job.x16);
        const size_t lo_off = (size_t)N * Kin;           // split arrays only

        // the previous item's loads into LDS, its stores and its LDS reads are
        // complete after this barrier (its fence waits for all memory counters)
        __syncthreads();
        if (tid < GM) {
            const int i = min(tid, nt - 1);
            int row;
            if (shared) {
                row = t_first + i;
            } else {
                const int p = job.perm[t_first + i];
                row = DOWN ? p : p / K;
            }
            s_arow[tid] = row;
        }
        __syncthreads();

        // weight rows of the item: gate rows 0..127 and up rows 128..255 of
        // the same moe_ff rows, or 256 down rows.  (The fields are selected
        // here, not in a lambda: a lambda that captured the argument struct
        // would copy it to private memory.)
        const WTensor &w0 = DOWN ? (shared ? job.sd : job.ed) : (shared ? job.sg : job.eg);
        const WTensor &w1 = DOWN ? (shared ? job.sd : job.ed) : (shared ? job.su : job.eu);
        const uint8_t *wb0 = w0.data + (size_t)e * w0.nb2 + (size_t)(rb * GN) * w0.nb1;
        const uint8_t *wb1 = w1.data + (size_t)e * w1.nb2 + (size_t)(rb * GN) * w1.nb1;
        const size_t wnb0 = w0.nb1, wnb1 = w1.nb1;
        // piece c = i * GT + tid of a tile (16 bytes at c * 16): row c >> 2,
        // slot c & 3, holding k-chunk (c & 3) ^ swz(row).  A wavefront's pieces
        // of one load are 1 KB of consecutive LDS, as the LDS-direct load writes.
        const uint8_t *ap[GP], *bp[GP];
#pragma unroll
        for (int i = 0; i < GP; i++) {
            const int c = i * GT + tid, row = c >> 2;
            const int q = (c & 3) ^ swz(row);
            ap[i] = reinterpret_cast<const uint8_t *>(A + (size_t)s_arow[row] * Kin) + q * 16;
            const bool up = !DOWN && row >= GN;
            bp[i] = (up ? wb1 + (size_t)(row - GN) * wnb1 : wb0 + (size_t)row * wnb0) + q * 16;
        }
        // stage st of the k loop into LDS buffer buf: 2 GP loads per thread
        // (none past the last stage, so nothing is in flight when the item ends)
        auto issue = [&](int st, int buf) {
            if (st >= total_steps) return;
            const int pass = st >= nsteps ? 1 : 0;
            const size_t kb = (size_t)(st - pass * nsteps) * GK * 2;
            const size_t ab = kb + (pass ? lo_off * 2 : 0);
#pragma unroll
            for (int i = 0; i < GP; i++) {
                const int dst = (i * GT + wave * 64) * 16;
                lds_load16(ap[i] + ab, &S[buf][0][dst]);
                lds_load16(bp[i] + kb, &S[buf][1][dst]);
            }
        };

        f4 acc[8][4];
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int tw = 0; tw < 4; tw++) acc[ti][tw] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
        for (int s0 = 0; s0 < GS - 1; s0++) issue(s0, s0);
        for (int st = 0; st < total_steps; st++) {
            const int buf = st % GS;
            // stage st has landed (the GS - 2 later stages may be in flight) in
            // this wavefront's pieces; the barrier makes that true of all, and
            // frees the buffer read in step st - 1 for stage st + GS - 1.  In
            // the last steps fewer stages follow: wait for all.
            if (st + GS - 2 < total_steps)
                GEMM_WAIT_VM(2 * GP * (GS - 2));
            else
                GEMM_WAIT_VM(0);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            issue(st + GS - 1, (st + GS - 1) % GS);
            h8 b[4];
#pragma unroll
            for (int tw = 0; tw < 4; tw++) b[tw] = *reinterpret_cast<const h8 *>(&S[buf][1][boff[tw]]);
#pragma unroll
            for (int ti = 0; ti < 8; ti++) {
                const h8 a = *reinterpret_cast<const h8 *>(&S[buf][0][aoff[ti]]);
#pragma unroll
                for (int tw = 0; tw < 4; tw++)
                    acc[ti][tw] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[tw], acc[ti][tw], 0, 0, 0);
            }
        }

        // results: output row of tile tw for lane r16; activation rows 16 ti + 4 g + i
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tt = tok0 + 16 * ti + 4 * g + i;
                if (tt >= nt) continue;
                if (!DOWN) {
#pragma unroll
                    for (int tj = 0; tj < 2; tj++) {
                        const int row = rb * GN + 32 * wq + 16 * tj + r16;
                        const float hv = gsilu(acc[ti][tj][i]) * acc[ti][2 + tj][i];
                        if (!shared) {
                            const int p = job.perm[t_first + tt];
                            job.h16[(size_t)p * FF + row] = f2h_rn(hv);
                        } else {
                            const int t = t_first + tt;
                            const uint16_t hi = f2h_rn(hv);
                            job.hs16[(size_t)t * SF + row] = hi;
                            job.hs16[(size_t)N * SF + (size_t)t * SF + row] =
                                f2h_rn(hv - (float)__builtin_bit_cast(_Float16, hi));
                        }
                    }
                } else {
                    float *o = shared ? job.ys + (size_t)(t_first + tt) * H
                                      : job.ye + (size_t)job.perm[t_first + tt] * H;
#pragma unroll
                    for (int tw = 0; tw < 4; tw++) o[rb * GN + brow[tw] + r16] = acc[ti][tw][i];
                }
            }
    }
}

// x (f32 rows) -> f16 rows, or the hi / lo f16 pair (lo rows after the hi rows)
__global__ __launch_bounds__(256) void k_cvt_f16(const float *__restrict__ src, size_t n, int split,
                                                 uint16_t *__restrict__ dst)
{
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    const float4 v = *reinterpret_cast<const float4 *>(src + i);
    const float x[4] = {v.x, v.y, v.z, v.w};
    uint16_t hi[4], lo[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        hi[k] = f2h_rn(x[k]);
        lo[k] = f2h_rn(x[k] - (float)__builtin_bit_cast(_Float16, hi[k]));
    }
    uint2 ph, pl;
    ph.x = (uint32_t)hi[0] | ((uint32_t)hi[1] << 16);
    ph.y = (uint32_t)hi[2] | ((uint32_t)hi[3] << 16);
    *reinterpret_cast<uint2 *>(dst + i) = ph;
    if (split) {
        pl.x = (uint32_t)lo[0] | ((uint32_t)lo[1] << 16);
        pl.y = (uint32_t)lo[2] | ((uint32_t)lo[3] << 16);
        *reinterpret_cast<uint2 *>(dst + n + i) = pl;
    }
}

hipError_t launch_cvt_f16(const float *src, int rows, int K, int split, uint16_t *dst, hipStream_t s)
{
    const size_t n = (size_t)rows * K;
    if (K % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_cvt_f16, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s, src, n, split, dst);
    return hipGetLastError();
}

bool gemm_shapes_ok(int H, int FF, int SF, bool shared)
{
    return H % GN_DN == 0 && H % GK == 0 && FF % GN_GU == 0 && FF % GK == 0 &&
           (!shared || (SF % GN_GU == 0 && SF % GK == 0));
}

hipError_t launch_gemm_f16(int phase, const GemmJob &job, hipStream_t s)
{
    if (!gemm_shapes_ok(job.H, job.FF, job.SF, job.has_shared)) return hipErrorInvalidValue;
    if (phase == 0)
        hipLaunchKernelGGL(k_gemm_f16<0>, dim3(GEMM_BLOCKS), dim3(GT), 0, s, job);
    else
        hipLaunchKernelGGL(k_gemm_f16<1>, dim3(GEMM_BLOCKS), dim3(GT), 0, s, job);
    return hipGetLastError();
}

} // namespace dmoe
