// attn.hip -- prefill-side neighbours of the W8A8 linears: the fused-QKV head
// split, the head merge and causal (optionally windowed) GQA attention.
//
// Reference: src/kernels/prefill_attention.cu.  The reference materialises the
// fp16 score matrix S = Q K^T [n_q, T, T] with a batched GEMM, runs a masked
// row softmax in place and a per-row S V product.  Here one kernel keeps
// 32-query tiles of query heads that share a KV head on chip and streams
// 32-key blocks of K and V through LDS, with the running-max (online) softmax,
// so the T x T matrix never reaches HBM.  Numerics follow the reference where they
// are observable: every score is rounded to fp16 before it is scaled
// (prefill_attention.cu:276-290 writes S in fp16, :160-162 reads it back),
// masked keys get weight 0, probabilities enter the V product as fp16 and the
// V product accumulates in fp32.  Only the order of fp32 sums and the point at
// which the weights are normalised (here after the V product, there before)
// differ; the tests bound the effect.
//
// Matrix-core mapping (v_mfma_f32_32x32x16_f16, one wave = 32 queries):
//   S^T[key][query] = K Q^T      A = K block from LDS   (row key,  k = d)
//                                B = Q tile, registers  (col query, k = d)
//   O^T[d][query]  += V^T P^T    A = V^T block from LDS (row d,    k = key)
//                                B = P^T, registers     (col query, k = key)
// For an A/B operand, lane l holds row/column l % 32 and k = 8 (l / 32) + 0..7;
// accumulator element i of lane l is row 8 (i / 4) + 4 (l / 32) + i % 4,
// column l % 32.  So after the score MFMAs each lane owns 16 keys of one
// query; its elements 0..7 and 8..15 are exactly the k slots the P^T operand
// needs for keys 0..15 and 16..31, with slot 8h + t <-> key
// 4h + t (t < 4) or 8 + 4h + (t - 4) (t >= 4).  The V^T operand is read from
// LDS in that same key order, so no lane exchange is needed between the two
// products; one lane swap (lane l <-> l ^ 32) gives the per-query maximum.
#include "common.h"

namespace fa {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int kAttnWaves = 4;      // (query head, tile) pairs per workgroup
constexpr int kAttnTile = 32;      // queries per wave and keys per block
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMasked = -1e30f;  // the reference's mask value (prefill_attention.cu:161)

__device__ __forceinline__ h8 ld_h8(const uint16_t* p) {
    return *reinterpret_cast<const h8*>(p);
}

// Position of key offset o (0..31) in a V^T row of LDS: within each 16-key
// group, position 8h + t holds key 4h + t (t < 4) or 8 + 4h + (t - 4)
// (t >= 4) -- the k-slot order of the P^T operand -- so one 16-byte LDS read
// gives a lane its 8 V^T slots.  Keys 2m and 2m + 1 land on adjacent
// positions.
__device__ __forceinline__ int vt_pos(int o) {
    return 16 * (o >> 4) + 8 * ((o & 7) >> 2) + 4 * ((o >> 3) & 1) + (o & 3);
}

// One workgroup: KV head `g` and four (query head, 32-query tile) pairs of
// its group -- four heads of one tile when the group size allows, else two
// heads x two tiles or one head x four tiles, so no wave idles for the
// DualAR (4 heads per group) or the DAC (1) layouts.  DP = head dim rounded
// up to 32 (D % 8 == 0, D <= DP).  The workgroup's key blocks (the union of
// its tiles' ranges; each wave skips blocks outside its own) are split in two
// halves: waves 0-3 take the first, waves 4-7 the second (each half with its
// own double-buffered K / V^T blocks in LDS and its own online softmax), and
// the halves are merged through LDS at the end.  Splitting the key range halves the serial chain of
// the tiles next to the diagonal of long sequences, which would otherwise
// set the kernel's duration.  Within a half, the block after next is in
// flight in registers while the current one is multiplied (one barrier per
// block), and V is transposed on its way into LDS: a thread loads the same
// 8 d of two adjacent keys and writes 8 packed key pairs.
template <int DP>
constexpr int attn_lds_bytes() {
    return 2 * 2 * (kAttnTile * (DP + 8) + DP * (kAttnTile + 8)) * 2;
}

template <int DP>
__global__ void __launch_bounds__(2 * kAttnWaves * 64, 1)
attention_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                 const uint16_t* __restrict__ v, uint16_t* __restrict__ out, int n_q, int n_kv,
                 int T, int D, float sm_scale, int window, int hpw, int R, int n_qb,
                 bool token_major) {
    constexpr int KS = DP + 8;            // K row stride in LDS (halves)
    constexpr int VS = kAttnTile + 8;     // V^T row stride in LDS (halves)
    constexpr int NC = 4 * DP;            // 16-byte chunks per block of K
    constexpr int NT = kAttnWaves * 64;   // threads per half
    constexpr int PT = (NC + NT - 1) / NT;
    constexpr int NU = 2 * DP;            // V units per block: key pair x 8 d
    constexpr int PV = (NU + NT - 1) / NT;
    constexpr int NKK = DP / 16;          // score MFMAs per block
    constexpr int NDB = DP / 32;          // d blocks of O^T
    constexpr int DC = DP / 8;            // K chunks per key
    constexpr int KB = kAttnTile * KS, VB = DP * VS;   // halves per K / V^T buffer
    extern __shared__ __align__(16) uint16_t lds[];

    const int half = threadIdx.x / NT;
    const int tid = threadIdx.x % NT, lane = tid & 63, wave = tid >> 6;
    uint16_t* const Ks = lds + half * 2 * (KB + VB);   // [2][KB]
    uint16_t* const Vs = Ks + 2 * KB;                 // [2][VB]
    const int col = lane & 31, hh = lane >> 5;
    // A workgroup covers hpw query heads of one KV group (hpw = 4, 2 or 1,
    // the largest that divides the group size) times R <= 4 / hpw consecutive
    // query tiles: wave w takes head w % hpw of its chunk and tile w / hpw
    // (waves past R tiles idle).
    const int gs = n_q / n_kv, chunks = gs / hpw;
    const int n_grp = (n_qb + R - 1) / R;
    // heaviest (last) tile groups first: they have the most key blocks
    const int grp = n_grp - 1 - (int)(blockIdx.x / (n_kv * chunks));
    const int rest = (int)(blockIdx.x % (n_kv * chunks));
    const int g = rest % n_kv, chunk = rest / n_kv;
    const int head = g * gs + chunk * hpw + wave % hpw;
    const int qt = grp * R + wave / hpw;             // this wave's query tile
    const bool active = wave / hpw < R && qt < n_qb;
    const int q0 = qt * kAttnTile;
    const int qi = q0 + col;                         // this lane's query

    const uint16_t* Kg = k + (int64_t)g * T * D;
    const uint16_t* Vg = v + (int64_t)g * T * D;

    // Q tile (B operand of the score product), zero past D and past T.
    h8 qf[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
        const int d = 16 * kk + 8 * hh;
        if (qi < T && d < D)
            qf[kk] = ld_h8(q + ((int64_t)head * T + qi) * D + d);
        else
            qf[kk] = h8{0, 0, 0, 0, 0, 0, 0, 0};
    }

    // key blocks of this wave's tile, and of the workgroup's (all its tiles)
    const int kb_hi = min(T - 1, q0 + kAttnTile - 1) / kAttnTile;
    const int kb_lo = (window > 0 ? max(0, q0 - window + 1) : 0) / kAttnTile;
    const int wg_q0 = grp * R * kAttnTile;
    const int wg_hi = min(T - 1, min(grp * R + R, n_qb) * kAttnTile - 1) / kAttnTile;
    const int wg_lo = (window > 0 ? max(0, wg_q0 - window + 1) : 0) / kAttnTile;
    const int left = window > 0 ? qi - window + 1 : 0;   // this lane's first key
    const float c1 = sm_scale * kLog2e;

    // Block loads are unconditional and their values are not touched until
    // the store one iteration later (so no wait follows the issue): a row
    // past T is read from row T - 1 (its scores are always masked: key >
    // every query, so its weight is exactly 0), and a 16-byte chunk past D
    // (DP > D) is read from the row start and zeroed at the store.
    h8 kr[PT], vr[PV][2];
    auto load_block = [&](int kb) {
#pragma unroll
        for (int p = 0; p < PT; ++p) {
            const int c = min(tid + p * NT, NC - 1);
            const int key = min(kb * kAttnTile + c / DC, T - 1), kd = 8 * (c % DC);
            kr[p] = ld_h8(Kg + (int64_t)key * D + (kd < D ? kd : 0));
        }
#pragma unroll
        for (int p = 0; p < PV; ++p) {
            const int u = min(tid + p * NT, NU - 1);
            const int key = kb * kAttnTile + 2 * (u & 15), vd = 8 * (u >> 4);
            const int off = vd < D ? vd : 0;
#pragma unroll
            for (int r = 0; r < 2; ++r)
                vr[p][r] = ld_h8(Vg + (int64_t)min(key + r, T - 1) * D + off);
        }
    };
    const h8 z8 = h8{0, 0, 0, 0, 0, 0, 0, 0};
    auto store_block = [&](int buf) {
#pragma unroll
        for (int p = 0; p < PT; ++p) {
            const int c = tid + p * NT;
            if (c < NC)
                *reinterpret_cast<h8*>(&Ks[buf * KB + (c / DC) * KS + 8 * (c % DC)]) =
                    (DP == 128 || 8 * (c % DC) < D) ? kr[p] : z8;
        }
#pragma unroll
        for (int p = 0; p < PV; ++p) {
            const int u = tid + p * NT;
            if (u < NU) {
                const int pos = vt_pos(2 * (u & 15)), vd = 8 * (u >> 4);
                const bool in = DP == 128 || vd < D;
                const h8 v0 = in ? vr[p][0] : z8, v1 = in ? vr[p][1] : z8;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    *reinterpret_cast<h2*>(&Vs[buf * VB + (vd + e) * VS + pos]) = h2{v0[e], v1[e]};
            }
        }
    };

    f16x acc_o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc_o[db][i] = 0.0f;
    // m_run: running maximum in units of score * sm_scale * log2(e); the
    // accumulators are rescaled only when a new maximum exceeds it by more
    // than 8 (probabilities relative to m_run then stay <= 2^8).
    float m_run = kMasked, l_run = 0.0f;

    // One 32-key block: scores, online softmax, V product.  `full`: every
    // key of the block is visible to all 32 queries of the tile (no mask).
    auto block = [&](int kb, int buf, bool full) {
        // every operand read of the block is issued up front: one LDS round
        // trip per block, the V^T reads complete under the softmax
        h8 ka[NKK], va[NDB][2];
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            ka[kk] = *reinterpret_cast<const h8*>(&Ks[buf * KB + col * KS + 16 * kk + 8 * hh]);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2)
                va[db][k2] = *reinterpret_cast<const h8*>(
                    &Vs[buf * VB + (32 * db + col) * VS + 16 * k2 + 8 * hh]);
        __builtin_amdgcn_sched_barrier(0);
        // S^T = K Q^T
        f16x s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[kk], qf[kk], s, 0, 0, 0);
        // scores rounded to fp16 (the reference stores S in fp16) and kept
        // packed: masked scores become -inf (weight exp2(-inf) = 0), the max
        // runs on packed halves and is taken before scaling (sm_scale > 0
        // keeps the order), and each weight is exp2(fma(float(s), c1, -m))
        // with the fp16 score as a mixed-precision fma operand.
        h2 sp[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) sp[j] = h2{(_Float16)s[2 * j], (_Float16)s[2 * j + 1]};
        if (!full) {
            const int kbase = kb * kAttnTile + 4 * hh;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int j = kbase + 8 * (i >> 2) + (i & 3);
                if (!(j <= qi && j >= left)) sp[i >> 1][i & 1] = -__builtin_inff16();
            }
        }
        h2 mx = __builtin_elementwise_max(__builtin_elementwise_max(sp[0], sp[1]),
                                          __builtin_elementwise_max(sp[2], sp[3]));
        mx = __builtin_elementwise_max(mx, __builtin_elementwise_max(
                                               __builtin_elementwise_max(sp[4], sp[5]),
                                               __builtin_elementwise_max(sp[6], sp[7])));
        float mloc = fmaxf((float)mx[0], (float)mx[1]);
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64)) * c1;
        const bool grow = mloc > m_run + 8.0f;
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - mloc) : 1.0f;
            m_run = grow ? mloc : m_run;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc_o[db][i] *= alpha;
        }
        h8 pb[2];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            pb[i >> 3][i & 7] = (_Float16)__builtin_amdgcn_exp2f(
                __builtin_fmaf((float)sp[i >> 1][i & 1], c1, -m_run));
        // l_run sums the fp16 weights the V product uses (v_dot2: exact pairs)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            l_run = __builtin_amdgcn_fdot2(
                h2{pb[i >> 2][2 * (i & 3)], pb[i >> 2][2 * (i & 3) + 1]}, h2{1, 1}, l_run, false);
        // O^T += V^T P^T
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2)
                acc_o[db] =
                    __builtin_amdgcn_mfma_f32_32x32x16_f16(va[db][k2], pb[k2], acc_o[db], 0, 0, 0);
    };

    // this half's key blocks: the first ceil(n / 2) of the tile's n blocks,
    // or the rest
    const int nkb = wg_hi - wg_lo + 1, n0 = (nkb + 1) / 2;
    const int my_lo = half ? wg_lo + n0 : wg_lo, my_n = half ? nkb - n0 : n0;
    if (my_n > 0) {
        load_block(my_lo);
        store_block(0);
    }
    __syncthreads();
    if (my_n > 1) load_block(my_lo + 1);
    for (int it = 0; it < n0; ++it) {
        const int kb = my_lo + it, buf = it & 1;
        if (it + 1 < my_n) {
            store_block(buf ^ 1);
            if (it + 2 < my_n) load_block(kb + 2);
        }
        if (active && it < my_n && kb >= kb_lo && kb <= kb_hi) {
            // every key of the block visible to all 32 queries of the tile
            const bool full = kb * kAttnTile + kAttnTile - 1 <= q0 &&
                              (window <= 0 || kb * kAttnTile >= q0 + kAttnTile - window);
            block(kb, buf, full);
        }
        __syncthreads();
    }

    // merge: the second half's waves leave (m, l, O^T) in LDS, lane-major
    // ([wave][value][lane] floats: conflict-free), the first half's combine
    // them with their own and write the output.
    constexpr int NV = 16 * NDB + 2;
    float* const red = reinterpret_cast<float*>(lds) + wave * NV * 64 + lane;
    if (half == 1 && active) {
        red[0] = m_run;
        red[64] = l_run;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) red[(2 + 16 * db + i) * 64] = acc_o[db][i];
    }
    __syncthreads();
    if (half == 1 || !active || qi >= T) return;
    const float m1 = red[0], m = fmaxf(m_run, m1);
    const float f0 = __builtin_amdgcn_exp2f(m_run - m), f1 = __builtin_amdgcn_exp2f(m1 - m);
    const float l_lane = l_run * f0 + red[64] * f1;
    const float l_tot = l_lane + __shfl_xor(l_lane, 32, 64);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    // head-major [n_q, T, D], or token-major [T, n_q D] (the merged layout
    // merge_heads would produce)
    uint16_t* orow = out + (token_major ? ((int64_t)qi * n_q + head) * D
                                        : ((int64_t)head * T + qi) * D);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int d = 32 * db + 8 * r + 4 * hh;
            if (d < D) {
                uint16_t o4[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int i = 4 * r + t;
                    const float o = acc_o[db][i] * f0 + red[(2 + 16 * db + i) * 64] * f1;
                    o4[t] = f2h(o * inv);
                }
                uint2 w;
                w.x = (uint32_t)o4[0] | ((uint32_t)o4[1] << 16);
                w.y = (uint32_t)o4[2] | ((uint32_t)o4[3] << 16);
                *reinterpret_cast<uint2*>(orow + d) = w;
            }
        }
}

// Any-shape attention (head dim not a multiple of 8 or above 128, a
// non-positive scale, or buffers not 16-byte aligned): one wave per (query
// head, query), two passes over the query's visible keys in blocks of 64,
// with the reference's operations (causal_softmax_kernel and sgemv_kernel,
// prefill_attention.cu:141-224, 325-349): scores float(fp16(q . k_j)) *
// scale; their max and exp-sum (one pass, the sum rescaled when the running
// max grows); then P = fp16(exp(v - max) * (1 / sum)) and
// O[d] = fp16(sum_j float(P_j) * float(V_jd)) with the fma chain in key order.
// A block's key rows are copied into the wave's LDS area 64 head-dim columns
// at a time with consecutive addresses (2-byte loads: any alignment), and
// lane j forms key j's dot product from there (rows padded to 66 halves, so
// the 64 lanes' reads fall in distinct banks); for O the lanes take head-dim
// columns of each V row.  Correct for every shape the API accepts; a
// fallback, not a fast path.
constexpr int kGenMaxD = 512;
constexpr int kGenRow = 66;      // LDS row stride of a staged key block (halves)

__global__ void __launch_bounds__(256)
attention_generic_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                         const uint16_t* __restrict__ v, uint16_t* __restrict__ out, int n_q,
                         int n_kv, int T, int D, float sm_scale, int window, bool token_major) {
    __shared__ uint16_t kblk[4][64 * kGenRow];
    __shared__ uint16_t qrow[4][kGenMaxD];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t idx = (int64_t)blockIdx.x * 4 + wave;
    if (idx >= (int64_t)n_q * T) return;          // whole wave; only wave-local LDS below
    const int head = (int)(idx / T), i = (int)(idx % T);
    const int g = head / (n_q / n_kv);
    const uint16_t* qr = q + ((int64_t)head * T + i) * D;
    const uint16_t* Kg = k + (int64_t)g * T * D;
    const uint16_t* Vg = v + (int64_t)g * T * D;
    const int left = window > 0 ? max(0, i - window + 1) : 0;
    uint16_t* kb = kblk[wave];
    uint16_t* qs = qrow[wave];
    for (int d = lane; d < D; d += 64) qs[d] = qr[d];
    // lane's score float(fp16(q . k_{j0 + lane})) * scale for the block at
    // j0 (rows past i read row i; their scores are not used).  A wave reads
    // back only LDS it wrote itself, in order: no barrier, only a wait.
    auto block_scores = [&](int j0) {
        float acc = 0.0f;
        for (int c0 = 0; c0 < D; c0 += 64) {
            const int cw = min(64, D - c0);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // earlier reads done
            const int cl = min(lane, cw - 1);
            for (int r0 = 0; r0 < 64; r0 += 16) {
                uint16_t kv[16];          // 16 loads in flight, then the writes
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    kv[r] = Kg[(int64_t)min(j0 + r0 + r, i) * D + c0 + cl];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (lane < cw) kb[(r0 + r) * kGenRow + lane] = kv[r];
            }
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            const uint16_t* row = kb + lane * kGenRow;
#pragma unroll 8
            for (int c = 0; c < cw; ++c)
                acc = __builtin_fmaf(h2f(qs[c0 + c]), h2f(row[c]), acc);
        }
        return h2f(f2h(acc)) * sm_scale;
    };
    // pass 1: running max and exp-sum over blocks (per block: its max, then
    // the sum rescaled to it)
    float m = -__builtin_inff(), l = 0.0f;
    for (int j0 = left; j0 <= i; j0 += 64) {
        const bool ok = j0 + lane <= i;
        const float s = block_scores(j0);
        const float bm = subgroup_max<64>(ok ? s : -__builtin_inff());
        const float mn = fmaxf(m, bm);
        float e = ok ? expf(s - mn) : 0.0f;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) e += __shfl_xor(e, off, 64);
        l = (m == mn ? l : l * expf(m - mn)) + e;
        m = mn;
    }
    const float mx = m;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    // pass 2: P and the key-ordered O chains
    constexpr int QR = kGenMaxD / 64;
    float o[QR];
#pragma unroll
    for (int r = 0; r < QR; ++r) o[r] = 0.0f;
    for (int j0 = left; j0 <= i; j0 += 64) {
        const float s = block_scores(j0);
        const float p = j0 + lane <= i ? h2f(f2h(expf(s - mx) * inv)) : 0.0f;
        const int nj = min(64, i - j0 + 1);
        // eight keys' V values in flight at a time (keys past i have P = 0
        // and read row i)
        for (int t0 = 0; t0 < nj; t0 += 8) {
#pragma unroll
            for (int r = 0; r < QR; ++r) {
                if (r * 64 >= D) continue;    // wave-uniform
                const int d = lane + 64 * r;
                const int dc = d < D ? d : D - 1;
                uint16_t vv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) vv[u] = Vg[(int64_t)min(j0 + t0 + u, i) * D + dc];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const float pj = __builtin_bit_cast(   // t0 + u is wave-uniform: a lane read
                        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), t0 + u));
                    o[r] = __builtin_fmaf(pj, h2f(vv[u]), o[r]);
                }
            }
        }
    }
    uint16_t* orow = out + (token_major ? ((int64_t)i * n_q + head) * D
                                        : ((int64_t)head * T + i) * D);
#pragma unroll
    for (int r = 0; r < QR; ++r) {
        const int d = lane + 64 * r;
        if (d < D) orow[d] = f2h(o[r]);
    }
}

// Fused QKV [T, (n_q + 2 n_kv) D] -> q [n_q, T, D], k / v [n_kv, T, D]; one
// thread per VEC halves (VEC = 8 when D % 8 == 0 and every buffer is 16-byte
// aligned, else 1).
template <int VEC>
__global__ void qkv_split_kernel(const uint16_t* __restrict__ qkv, uint16_t* __restrict__ q,
                                 uint16_t* __restrict__ k, uint16_t* __restrict__ v, int T,
                                 int n_q, int n_kv, int D) {
    typedef uint16_t u16v __attribute__((ext_vector_type(VEC)));
    const int DV = D / VEC;
    const int64_t total = (int64_t)T * (n_q + 2 * n_kv) * DV;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    // source order: consecutive threads read consecutive chunks of one token row
    const int dv = (int)(idx % DV);
    const int64_t r = idx / DV;
    const int slot = (int)(r % (n_q + 2 * n_kv));
    const int t = (int)(r / (n_q + 2 * n_kv));
    const u16v x = *reinterpret_cast<const u16v*>(qkv + idx * VEC);
    uint16_t* dst;
    if (slot < n_q)
        dst = q + ((int64_t)slot * T + t) * D;
    else if (slot < n_q + n_kv)
        dst = k + ((int64_t)(slot - n_q) * T + t) * D;
    else
        dst = v + ((int64_t)(slot - n_q - n_kv) * T + t) * D;
    *reinterpret_cast<u16v*>(dst + dv * VEC) = x;
}

// Head-major [H, T, D] -> token-major [T, H D].
template <int VEC>
__global__ void merge_heads_kernel(const uint16_t* __restrict__ heads, uint16_t* __restrict__ out,
                                   int T, int H, int D) {
    typedef uint16_t u16v __attribute__((ext_vector_type(VEC)));
    const int DV = D / VEC;
    const int64_t total = (int64_t)T * H * DV;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    // destination order: consecutive threads write consecutive chunks of a token row
    const int dv = (int)(idx % DV);
    const int64_t r = idx / DV;
    const int h = (int)(r % H);
    const int t = (int)(r / H);
    *reinterpret_cast<u16v*>(out + idx * VEC) =
        *reinterpret_cast<const u16v*>(heads + ((int64_t)h * T + t) * D + dv * VEC);
}

inline unsigned blocks_for(int64_t n, int threads) {
    return (unsigned)((n + threads - 1) / threads);
}

template <int DP>
hipError_t launch_attention(dim3 grid, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            uint16_t* out, int n_q, int n_kv, int T, int D, float sm_scale,
                            int window, int hpw, int R, int n_qb, bool token_major,
                            hipStream_t stream) {
    constexpr int lds = attn_lds_bytes<DP>();
    static_assert(lds >= 4 * 64 * (DP / 2 + 2) * 4, "merge area exceeds the block buffers");
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&attention_kernel<DP>),
        hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return attr;
    attention_kernel<DP><<<grid, 2 * kAttnWaves * 64, lds, stream>>>(
        q, k, v, out, n_q, n_kv, T, D, sm_scale, window, hpw, R, n_qb, token_major);
    return hipGetLastError();
}

}  // namespace

int attention_padded_dim(int D) { return D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 0; }

int attention_max_dim() { return kGenMaxD; }

hipError_t launch_prefill_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                    uint16_t* out, int n_q, int n_kv, int T, int D, float sm_scale,
                                    int window, bool token_major, hipStream_t stream) {
    const bool fast = D % 8 == 0 && attention_padded_dim(D) != 0 && sm_scale > 0.0f &&
                      (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15) == 0;
    if (!fast) {
        const int64_t rows = (int64_t)n_q * T;
        attention_generic_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, stream>>>(
            q, k, v, out, n_q, n_kv, T, D, sm_scale, window, token_major);
        return hipGetLastError();
    }
    const int gs = n_q / n_kv;
    const int hpw = gs % 4 == 0 ? 4 : gs % 2 == 0 ? 2 : 1;   // heads per workgroup
    const int n_qb = (T + kAttnTile - 1) / kAttnTile;
    // query tiles per workgroup: fill all four wave slots unless that leaves
    // fewer workgroups than CUs (measured: MHA with 8 heads at T = 1024 is
    // faster with idle waves and 4x the workgroups)
    int R = kAttnWaves / hpw;
    auto wgs = [&](int r) { return (int64_t)((n_qb + r - 1) / r) * n_kv * (gs / hpw); };
    while (R > 1 && wgs(R) < 256) R /= 2;
    const dim3 grid((unsigned)wgs(R));
    switch (attention_padded_dim(D)) {
        case 32:
            return launch_attention<32>(grid, q, k, v, out, n_q, n_kv, T, D, sm_scale, window,
                                        hpw, R, n_qb, token_major, stream);
        case 64:
            return launch_attention<64>(grid, q, k, v, out, n_q, n_kv, T, D, sm_scale, window,
                                        hpw, R, n_qb, token_major, stream);
        case 128:
            return launch_attention<128>(grid, q, k, v, out, n_q, n_kv, T, D, sm_scale, window,
                                         hpw, R, n_qb, token_major, stream);
        default:
            return hipErrorInvalidValue;
    }
}

hipError_t launch_qkv_split(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v, int T,
                            int n_q, int n_kv, int D, bool vec, hipStream_t stream) {
    const int64_t rows = (int64_t)T * (n_q + 2 * n_kv);
    if (vec)
        qkv_split_kernel<8><<<blocks_for(rows * (D / 8), 256), 256, 0, stream>>>(qkv, q, k, v, T,
                                                                               n_q, n_kv, D);
    else
        qkv_split_kernel<1><<<blocks_for(rows * D, 256), 256, 0, stream>>>(qkv, q, k, v, T, n_q,
                                                                         n_kv, D);
    return hipGetLastError();
}

hipError_t launch_merge_heads(const uint16_t* heads, uint16_t* out, int T, int H, int D, bool vec,
                              hipStream_t stream) {
    const int64_t rows = (int64_t)T * H;
    if (vec)
        merge_heads_kernel<8><<<blocks_for(rows * (D / 8), 256), 256, 0, stream>>>(heads, out, T,
                                                                                 H, D);
    else
        merge_heads_kernel<1><<<blocks_for(rows * D, 256), 256, 0, stream>>>(heads, out, T, H, D);
    return hipGetLastError();
}

}  // namespace fa
