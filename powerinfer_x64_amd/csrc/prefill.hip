// prefill.hip -- causal GQA flash attention for a whole prompt (gfx950 MFMA).
//
// Replaces the reference's prefill attention, which runs the decode loop once
// per prompt token (src/model/mod.rs:668 token loop, :1140-1190 append-then-
// attend), i.e. row i attends keys 0..i.
//
// Head dim 128 runs prefill_fa_kernel (below), head dim 256 prefill_fa256_kernel
// (16 query rows per wavefront, the same two-phase schedule).
//
// prefill_fa_kernel: a workgroup of 8 wavefronts covers
// HPW query heads that share one KV head and 256/HPW query positions; each
// wavefront owns 32 query rows of one head and computes, per 64-key tile,
//   S^T[64 key x 32 q] = K . Q^T          (16 x v_mfma_f32_32x32x16)
//   O^T[D x 32 q]     += V^T . P^T        (16 x v_mfma_f32_32x32x16)
// with the softmax in f32 on S^T, where a lane owns one query column, so the
// row max / sum need one cross-lane step.  Tiles past the diagonal are
// skipped; workgroups are launched heaviest-first.
//
// gfx950 facts the schedule is built on (measured with in-kernel timers):
// within one wavefront an MFMA followed by v_exp serialises, while the MFMAs
// of one wavefront and the VALU work of another on the same SIMD overlap; a
// v_dot2 queues behind the other wavefront's MFMAs; LDS serves one wave64
// read per ~4 clocks (256 B/clk for 16-byte reads).  So each wavefront
// alternates a pure MFMA phase and a pure VALU (softmax) phase, and the two
// wavefronts of a SIMD run in opposite phases.
#include <cstdlib>

#include "pi_device.hpp"
#include "pi_launch.hpp"

namespace pi {
namespace {

constexpr int BN = 64;         // keys per block
constexpr int ROWS = 32;       // query rows per wavefront
// The running max of a row moves only when a lane's exps of a tile against it sum past
// kSumCap = 2^13 (an overflow to inf or a NaN counts too): the tile's max is then taken and
// the tile redone against it.  With at most 32 exps per lane, a sum within the cap means
// no score exceeded the max by more than 13 (log2 units), so every P value stays below
// 2^13, far inside the f32 / bf16 range; a sum past it means one exceeded it by more than 8
// (or 9 at 16 exps per lane).  Most tiles take no max at all; the first tile of a row always
// moves it (from -1e30).
constexpr float kSumCap = 8192.0f;

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16> {
    typedef bf16x8 v8;
    typedef bf16x4 v4;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mfma<f16> {
    typedef f16x8 v8;
    typedef f16x4 v4;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

struct PrefillArgs {
    const void* q;
    const void* k;
    const void* v;
    float* out;
    int S;      // query rows per sequence
    int Sk;     // keys per sequence (K / V rows)
    int q_off;  // position of query row 0 among the keys (causal: row i sees keys <= q_off + i)
    int hq, hkv, group, causal, gqa_mode;
    float qk_scale;  // scale * log2(e)
    // causal balance: workgroup y takes query blocks nqb-1-y and y in turn, so
    // every workgroup walks nqb + 1 key tiles and one wave of workgroups fills
    // the chip evenly (else: one block each, heaviest first)
    int paired;
    // key split (a launch with fewer workgroups than CUs): blockIdx.z = batch * ksplit +
    // split.  A query block of n <= kthr key tiles is not split: split 0 takes all its
    // tiles and writes the output, the other splits skip it.  A longer one runs in
    // split_pieces(n) = min(ksplit, ceil(n / kthr)) pieces: piece k takes tiles [k p,
    // (k+1) p), p = ceil(n / pieces), and leaves its unnormalised O and (max, sum) for
    // prefill_merge_kernel; splits past the block's pieces skip it.
    int ksplit;
    int kthr;
    float* part_o;   // [ksplit][B][S][Hq][D]
    float* part_ml;  // [ksplit][B][S][Hq][2]
    // optional output gate [B][S][Hq][D]: out *= 1 / (1 + exp(-gate)) (src/model/mod.rs:1192-1196),
    // applied where the normalised output is written (the epilogue, or the merge of key splits)
    const float* gate;
    // Paged source (prefill_fa_kernel<., ., ., true>, one sequence): K / V out of the pool's
    // page blocks through the page-table row pt (kpool / vpool + (page * hkv + kv head) *
    // kstride / vstride bytes), and q in f32 when q_f32 (else in T).
    const int32_t* pt;
    const char* kpool;
    const char* vpool;
    size_t kstride, vstride;
    int n_pages;
    int q_f32;
};

__device__ __forceinline__ float gate_sigmoid(float g) { return 1.0f / (1.0f + expf(-g)); }

// Pieces of a query block of n key tiles under a key split (1: the block runs whole).
__host__ __device__ __forceinline__ int split_pieces(int n, int ksplit, int kthr) {
    return ksplit > 1 && kthr > 0 && n > kthr ? min(ksplit, (n + kthr - 1) / kthr) : 1;
}

__device__ __forceinline__ int head_of(int kvh, int c, int hkv, int group, int mode) {
    return mode == 0 ? kvh + c * hkv : kvh * group + c;
}

// ---------------------------------------------------------------------------
// prefill_fa_kernel: 8 wavefronts per workgroup (2 per SIMD), one workgroup
// per CU.  Wave w owns 32 query rows of one query head: head slot w % HPW of
// the workgroup's HPW heads (they share one KV head) and row tile w / HPW, so
// a workgroup covers HPW heads x 256/HPW rows and every K/V byte it stages in
// LDS serves 8 wavefronts.
//
// A "unit" u holds K of tile u and V of tile u - 1 in one of four LDS
// buffers; it arrives by direct global -> LDS loads (no registers, no LDS
// stores): K in [key][dim] order with 272-byte rows, V in [key][dim] order
// with 256-byte rows whose 16-byte chunks are XOR-swizzled by row.  K
// fragments are 16-byte reads; V^T fragments come from two transposing reads
// (ds_read_b64_tr_b16).  All fragment reads are conflict-free and run PF
// ahead of their MFMAs.  Only a wavefront's last tile can need the causal /
// prompt-end mask; the mask is one wave-uniform branch around a straight-line
// select block.
// ---------------------------------------------------------------------------
// Three-way max as one v_max3_f32.  fmaxf would first quiet a signalling NaN in every
// operand (an extra v_max per score); scores come from MFMA accumulators or -inf masks,
// never a signalling NaN, so the plain instruction gives the same result.
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float max32(const f32x16& s, const f32x16& t) {
    const float a = vmax3(s[0], s[1], s[2]), b = vmax3(s[3], s[4], s[5]);
    const float c = vmax3(s[6], s[7], s[8]), d = vmax3(s[9], s[10], s[11]);
    const float e = vmax3(s[12], s[13], s[14]), f = vmax3(s[15], t[0], t[1]);
    const float g = vmax3(t[2], t[3], t[4]), h = vmax3(t[5], t[6], t[7]);
    const float i = vmax3(t[8], t[9], t[10]), j = vmax3(t[11], t[12], t[13]);
    const float k = vmax3(a, b, c), l = vmax3(d, e, f), m = vmax3(g, h, i);
    return vmax3(vmax3(k, l, m), j, vmax3(t[14], t[15], j));
}

// Head dims 128 and 256.  D = 128: 8 wavefronts (two per SIMD, in opposite
// phases, see below) and four unit buffers.  D = 256: O and Q^T take 192
// registers at 32 query rows, so the workgroup has 4 wavefronts (one per SIMD,
// up to 512 registers each) and two unit buffers; each wavefront runs its MFMA
// and softmax phases back to back.
template <int D> struct PrefillCfg;
template <> struct PrefillCfg<64> { static constexpr int NW = 8, NB = 4; };
template <> struct PrefillCfg<128> { static constexpr int NW = 8, NB = 4; };
template <> struct PrefillCfg<256> { static constexpr int NW = 4, NB = 2; };

template <typename T, int HPW, int D, bool PG>
__global__ __launch_bounds__(64 * PrefillCfg<D>::NW, 1) void prefill_fa_kernel(PrefillArgs a) {
    typedef typename Mfma<T>::v8 v8;
    typedef typename Mfma<T>::v4 v4;
    typedef short s4 __attribute__((ext_vector_type(4)));
    constexpr int NW = PrefillCfg<D>::NW;
    constexpr int RT = NW / HPW;      // row tiles per workgroup
    constexpr int WROWS = ROWS * RT;  // query rows per workgroup
    constexpr int NB = PrefillCfg<D>::NB;  // unit buffers
    constexpr int NDT = D / 32;       // 32-dim tiles of O^T
    constexpr int KS = D + 8;         // K [key][dim] row stride (elements): 16 bytes of padding
    constexpr int KCH = KS / 8;       // 16-byte chunks per K row (17 or 33)
    // direct loads of 1 KB per K tile: 17 or 33 padded rows; paged, D / 8 (one per 16-byte chunk)
    constexpr int K_INSTR = PG ? D / 8 : BN * KCH / 64;
    constexpr int KJ = (K_INSTR + NW - 1) / NW;  // K loads per wavefront
    constexpr int V_INSTR = BN * D * 2 / 1024;  // direct loads of 1 KB per V tile (16 or 32)
    constexpr int VJ = V_INSTR / NW;  // V loads per wavefront
    constexpr int VRPI = 1024 / (2 * D);  // V rows per load (4 or 2)
    constexpr int VCPR = D / 8;       // 16-byte chunks per V row (8, 16 or 32)
    // contiguous V rows: the 32-dim group of a chunk is XORed with the row's low bits (two
    // at D >= 128, one at D = 64, whose rows hold two groups)
    constexpr int VSW = NDT >= 4 ? 3 : 1;
    // buffer u % NB holds K of tile u and V of tile u - 1.  Contiguous source: K [key][dim] with
    // padded rows, V [key][dim] with 2D-byte rows, chunk c of row r at c ^ 4*(r % 4) (c ^ 4*(r % 2) at D = 64).  Paged
    // source, page-major like the pool's blocks: K [4 pages][D/8][16 keys][8] with key pi(s)
    // in slot s (pi swaps bits 2 and 3), V [4 pages][D][16 keys] with the 8-key halves of
    // dim d's 32-byte row swapped when bit 2 ^ bit 3 of d is set (16 consecutive dims then
    // cover every bank once).
    __shared__ __attribute__((aligned(1024))) T sk[NB][BN * KS];
    __shared__ __attribute__((aligned(1024))) T sv[NB][BN * D];

    {  // a head that does not exist (modulo map with n_q_heads not a multiple of n_kv_heads:
       // HPW is 1) makes the whole workgroup leave, before any barrier
        const int per_kv = a.group / HPW;
        const int hs0 = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) % HPW;
        if (head_of((int)blockIdx.x / per_kv, ((int)blockIdx.x % per_kv) * HPW + hs0, a.hkv,
                    a.group, a.gqa_mode) >= a.hq)
            return;
    }
    const int nqb = (a.S + WROWS - 1) / WROWS;
    const int by = blockIdx.y;
    const int n_blocks = a.paired && by != nqb - 1 - by ? 2 : 1;
    for (int blk = 0; blk < n_blocks; ++blk) {
    // heaviest (latest) query blocks first; a paired workgroup then takes block y
    int qb = blk == 0 ? (a.paired ? nqb - 1 - by : (int)gridDim.y - 1 - by) : by;
    if (blk > 0) {
        // every wave is past its last LDS read of the previous block before the
        // new block's loads land in the unit buffers
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }
    // Everything below is derived afresh for each block from values the compiler
    // cannot carry over (opaque copies), so nothing stays live across blocks.
    int tid = threadIdx.x, bxx = blockIdx.x;
    asm volatile("" : "+v"(tid));
    asm volatile("" : "+s"(bxx), "+s"(qb));
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hs = wave % HPW, rt = wave / HPW;
    const int b = (int)blockIdx.z / a.ksplit, ksp = (int)blockIdx.z % a.ksplit;
    const int S = a.S, Sk = a.Sk, q_off = a.q_off;
    const int per_kv = a.group / HPW;           // workgroups per KV head
    const int kvh = bxx / per_kv;
    const int head = head_of(kvh, (bxx % per_kv) * HPW + hs, a.hkv, a.group, a.gqa_mode);
    const int p0 = qb * WROWS + rt * ROWS;
    const int wg_keys = a.causal ? min(Sk, q_off + qb * WROWS + WROWS) : Sk;
    const int n_tiles = (wg_keys + BN - 1) / BN;
    // this workgroup's key tiles: [tb, tb + nloc); step t below works on tile tb + t
    const int pieces = split_pieces(n_tiles, a.ksplit, a.kthr);
    if (ksp >= pieces) continue;  // uniform per workgroup
    const bool split = pieces > 1;
    const int kper = (n_tiles + pieces - 1) / pieces;
    const int tb = min(n_tiles, ksp * kper);
    const int nloc = min(n_tiles, tb + kper) - tb;
    const int w_keys = a.causal ? min(Sk, q_off + p0 + ROWS) : Sk;
    const int w_tiles = p0 < S ? (w_keys + BN - 1) / BN : 0;  // tiles this wavefront attends
    // Tiles from t_mask on hold a key past the wavefront's first row (causal)
    // or past the keys; they go through the mask.  Without an offset that is
    // at most the last tile; with one, the last two.
    const int t_mask = min(a.causal ? (q_off + p0 + 1) / BN : Sk / BN, Sk / BN);

    const int r = lane & 31;   // query column of this lane
    const int hh = lane >> 5;  // 8-wide k slice of the MFMA operands
    const int qpos = p0 + r;

    // Q^T operand: lane holds q[qpos][16*kk + 8*hh .. +7]
    v8 qr[D / 16];
    if (PG && a.q_f32) {  // f32 query rows, rounded to T here (RNE)
        const float* qg = reinterpret_cast<const float*>(a.q);
        const bool ok = qpos < S;
        const float* qrow = qg + (((size_t)b * S + (ok ? qpos : 0)) * a.hq + head) * D;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
            const f32x4 lo = *reinterpret_cast<const f32x4*>(qrow + 16 * kk + 8 * hh);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(qrow + 16 * kk + 8 * hh + 4);
            v8 t = {(T)lo[0], (T)lo[1], (T)lo[2], (T)lo[3], (T)hi[0], (T)hi[1], (T)hi[2], (T)hi[3]};
            if (!ok) t = v8{};
            qr[kk] = t;
        }
    } else {
        const T* qg = reinterpret_cast<const T*>(a.q);
        const bool ok = qpos < S;
        const T* qrow = qg + (((size_t)b * S + (ok ? qpos : 0)) * a.hq + head) * D;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
            v8 t = *reinterpret_cast<const v8*>(qrow + 16 * kk + 8 * hh);
            if (!ok) t = v8{};
            qr[kk] = t;
        }
    }
    f32x16 o[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) o[i] = f32x16{};
    float m_run = -1e30f, l_run = 0.f;

    const size_t tok_stride = (size_t)a.hkv * D;
    const T* kbase = reinterpret_cast<const T*>(a.k) + ((size_t)b * Sk * a.hkv + kvh) * D;
    const T* vbase = reinterpret_cast<const T*>(a.v) + ((size_t)b * Sk * a.hkv + kvh) * D;

    // Direct global -> LDS loads (16 bytes per lane, lane i lands at base +
    // 16 i).  K: load i of a tile covers chunks 64 i .. 64 i + 63 of the padded
    // tile (row = chunk / 17; chunk 16 of a row is padding and reloads chunk
    // 0).  V: load i covers rows 4 i .. 4 i + 3.  Rows past the prompt reload
    // row Sk-1 (finite values; their scores are masked to -inf, P = 0).
    typedef __attribute__((address_space(3))) void lds_void;
    // The load is issued from inline assembly so that the compiler does not
    // add vmcnt waits before LDS reads (it cannot tell the buffers apart);
    // the kernel waits for each unit explicitly before the barrier that
    // publishes it.
    // M0 (the LDS destination) is a register the compiler reserves, so the
    // assembly saves and restores it around the load.
    auto dma16 = [](const void* src, lds_void* dst) {
        unsigned lds = (unsigned)(uintptr_t)dst;
        if constexpr (D == 256) lds = __builtin_amdgcn_readfirstlane(lds);
        unsigned saved;
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\t"
                     "global_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(src), "s"(lds) : "memory");
    };
    // scalar base + 32-bit lane byte offset form, for the common full tile.
    // The base and the LDS address are wave-uniform; at D = 256 the compiler
    // would otherwise hand the base over in vector registers, so readfirstlane
    // pins both to scalar registers, as the instruction requires.
    auto dma16s = [](const void* base, unsigned voff, lds_void* dst) {
        unsigned lds = (unsigned)(uintptr_t)dst;
        if constexpr (D == 256) {
            const uintptr_t bp = (uintptr_t)base;
            const unsigned blo = __builtin_amdgcn_readfirstlane((unsigned)bp);
            const unsigned bhi = __builtin_amdgcn_readfirstlane((unsigned)(bp >> 32));
            base = (const void*)(((uintptr_t)bhi << 32) | blo);
            lds = __builtin_amdgcn_readfirstlane(lds);
        }
        unsigned saved;
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\t"
                     "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(voff), "s"(base), "s"(lds) : "memory");
    };
    // this lane's row and byte offset (within a tile) for each of its loads
    int k_row[KJ], v_row[VJ];
    unsigned k_off[KJ], v_off[VJ];
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
        const int i = wave + NW * j;
        const int L = 64 * (i < K_INSTR ? i : 0) + lane;
        const int row = L / KCH, ch = L - row * KCH;
        k_row[j] = row;
        k_off[j] = (unsigned)(((size_t)row * tok_stride + 8 * (ch < KCH - 1 ? ch : 0)) * sizeof(T));
    }
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
        const int i = VJ * wave + j;
        const int row = VRPI * i + lane / VCPR;
        const int cc = (lane % VCPR) ^ (4 * (row & VSW));
        v_row[j] = row;
        v_off[j] = (unsigned)(((size_t)row * tok_stride + 8 * cc) * sizeof(T));
    }
    auto issue_unit_c = [&](int u) {
        const int buf = u % NB;
        const int k0 = (tb + u) * BN;
        if (k0 + BN <= Sk) {
            const T* kb = kbase + (size_t)k0 * tok_stride;
#pragma unroll
            for (int j = 0; j < KJ; ++j) {
                const int i = wave + NW * j;
                if (i < K_INSTR) dma16s(kb, k_off[j], (lds_void*)&sk[buf][512 * i]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < KJ; ++j) {
                const int i = wave + NW * j;
                if (i < K_INSTR) {
                    const int key = min(k0 + k_row[j], Sk - 1);
                    const T* src = kbase + (size_t)key * tok_stride +
                                   (k_off[j] - (size_t)k_row[j] * tok_stride * sizeof(T)) / sizeof(T);
                    dma16(src, (lds_void*)&sk[buf][512 * i]);
                }
            }
        }
        if (u >= 1) {
            const int v0 = k0 - BN;
            const T* vb = vbase + (size_t)v0 * tok_stride;
            if (v0 + BN <= Sk) {
#pragma unroll
                for (int j = 0; j < VJ; ++j) dma16s(vb, v_off[j], (lds_void*)&sv[buf][512 * (VJ * wave + j)]);
            } else {
#pragma unroll
                for (int j = 0; j < VJ; ++j) {
                    const int key = min(v0 + v_row[j], Sk - 1);
                    const T* src = vbase + (size_t)key * tok_stride +
                                   (v_off[j] - (size_t)v_row[j] * tok_stride * sizeof(T)) / sizeof(T);
                    dma16(src, (lds_void*)&sv[buf][512 * (VJ * wave + j)]);
                }
            }
        }
    };
    // Paged source.  The page ids of a tile's four 16-key pages (pages past the sequence's
    // last key repeat its last page; the keys there are masked) are scalar loads: a vector
    // load would share vmcnt with the direct loads in flight (its wait would drain them all).  A page id outside [0, n_pages) holds
    // no tokens: page 0 is read in its place and its keys are masked (bit j of the unit's bad
    // mask), as the decode does.  Load i of a unit moves 1 KB of one page, i / NDT: K chunks
    // 4 (i % NDT) .. +3, V dims 32 (i % NDT) .. +31.  With i = wave + NW j and NW a multiple
    // of NDT, a wave's loads keep one 1 KB slice (i % NDT) of pages wave / NDT + (NW / NDT) j:
    // the base is one scalar per load and the lane offsets are fixed.
    typedef int i32x4_ __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(4))) const int32_t* const_i32p;
    typedef __attribute__((address_space(4))) const i32x4_* const_i32x4p;
    const int last_pg = (Sk - 1) >> 4;
    const int pj0 = wave / NDT, pq = wave % NDT;
    // a page's blocks of all KV heads span under 4 GB (checked by the launcher)
    const unsigned page_bytes_k = (unsigned)(a.hkv * a.kstride), page_bytes_v = (unsigned)(a.hkv * a.vstride);
    const char* kq_pg = a.kpool + (size_t)kvh * a.kstride + 1024 * pq;
    const char* vq_pg = a.vpool + (size_t)kvh * a.vstride + 1024 * pq;
    // K: lane l is key slot l % 16 (holding key pi(l % 16), pi swapping bits 2 and 3) of
    // chunk 4 (i % NDT) + l / 16.  V: lane l is the 8-key half (l % 2) ^ g(d) of dim
    // d = 32 (i % NDT) + l / 2, g(d) = bit 2 ^ bit 3 of d.
    const int ks_ = lane & 15;
    const unsigned k_lo = (unsigned)((lane >> 4) * 256 + 16 * ((ks_ & 3) | ((ks_ & 4) << 1) | ((ks_ & 8) >> 1)));
    const int vd_ = lane >> 1;
    const unsigned v_lo = (unsigned)(vd_ * 32 + 16 * ((lane & 1) ^ (((vd_ >> 2) ^ (vd_ >> 3)) & 1)));
    // Paged, 8 wavefronts: the lead wave w (0-3) issues the loads of waves w and w + 4 (its
    // lag partner's share) after its softmax, when its lag partner runs its MFMA phase; the
    // lag waves then issue none and their path through a step (softmax, MFMA phase) is free
    // of load issue, which stalls on the direct-load path's latency.
    constexpr int LPD = (PG && NW == 8) ? 2 : 1;  // load passes of a loading wave
    const bool loader = wave < NW / LPD;
    // this wave's page ids for the K tile of the unit issued last (the next unit's V tile)
    unsigned koff_prev[LPD][KJ] = {};
    auto load_ids = [&](int u) {
        i32x4_ r = {};
        if constexpr (PG) {
            const int p0_ = (tb + u) * (BN >> 4);
            if (p0_ + 3 <= last_pg) {
                r = *(const_i32x4p)((const_i32p)a.pt + __builtin_amdgcn_readfirstlane(p0_));
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    r[j] = ((const_i32p)a.pt)[__builtin_amdgcn_readfirstlane(min(p0_ + j, last_pg))];
            }
        }
        return r;
    };
    // Whether every page id of this workgroup's tiles lies in the pool, checked once before
    // any direct load (so its vector loads' wait drains nothing): then no unit needs a
    // bad-page mask and only the loading waves read page ids.
    bool ids_ok = true;
    if constexpr (PG) {
        const int pe = min((tb + nloc) * (BN >> 4), last_pg + 1);
        bool bad_l = false;
        for (int pp = tb * (BN >> 4) + lane; pp < pe; pp += 64)
            bad_l |= (unsigned)a.pt[pp] >= (unsigned)a.n_pages;
        ids_ok = !__any(bad_l);
    }
    // the loading waves read the next unit's ids at the start of an issue, so the scalar
    // load's latency passes while this unit's direct loads issue
    i32x4_ ids_next = loader ? load_ids(0) : i32x4_{};
    unsigned bad_units = 0;   // 4 bits per unit buffer: the K tile's pages outside the pool
    auto issue_unit_p = [&](int u) {
        const int buf = u % NB;
        i32x4_ r;
        if (loader) {
            r = ids_next;
            ids_next = load_ids(u + 1);
        } else {
            if (ids_ok) return;
            r = load_ids(u);
        }
        if (!ids_ok) {
            unsigned bad = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) bad |= (unsigned)((unsigned)r[j] >= (unsigned)a.n_pages) << j;
            bad_units = (bad_units & ~(15u << (4 * buf))) | (bad << (4 * buf));
        }
        if (!loader) return;
#pragma unroll
        for (int ps = 0; ps < LPD; ++ps) {
            const int wv = wave + ps * (NW / LPD);  // the wave whose share this is
            unsigned koff[KJ];
#pragma unroll
            for (int j = 0; j < KJ; ++j) {
                const int pj = wv / NDT + (NW / NDT) * j;
                const int x = pj == 0 ? r[0] : pj == 1 ? r[1] : pj == 2 ? r[2] : r[3];
                koff[j] = (unsigned)x < (unsigned)a.n_pages ? (unsigned)x : 0u;
                const int i = wv + NW * j;
                if (i < K_INSTR)
                    dma16s(kq_pg + (size_t)koff[j] * page_bytes_k, k_lo, (lds_void*)&sk[buf][512 * i]);
            }
            if (u >= 1) {
#pragma unroll
                for (int j = 0; j < KJ; ++j) {
                    const int i = wv + NW * j;
                    if (i < K_INSTR)
                        dma16s(vq_pg + (size_t)koff_prev[ps][j] * page_bytes_v, v_lo, (lds_void*)&sv[buf][512 * i]);
                }
            }
#pragma unroll
            for (int j = 0; j < KJ; ++j) koff_prev[ps][j] = koff[j];
        }
    };
    auto issue_unit = [&](int u) {
        if constexpr (PG) issue_unit_p(u);
        else issue_unit_c(u);
    };
    // barrier without the compiler's fence: LDS visibility is handled by the
    // explicit waits; the empty asm keeps memory accesses on their side
    auto barrier = [&]() {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    const float c = a.qk_scale;
    typedef __attribute__((address_space(3))) const T* lds_ptr;
    typedef __attribute__((address_space(3))) const v8* lds_v8;
    typedef __attribute__((address_space(3))) s4* lds_s4;
    // Paged source: the K operand's row r reads key r with bits 2 and 3 swapped (key slot
    // r % 16 of page r / 16 holds it), so slot e of a lane's P^T operand (built from the S^T
    // accumulator, rows 8 j + 4 hh + e % 4) is key 8 hh + e of its 16-key step: the V^T
    // operand is then 8 consecutive keys of one dim, one 16-byte read of the page's V rows.
    const lds_ptr k_lane = PG ? (lds_ptr)&sk[0][(r >> 4) * 16 * D + hh * 128 + (r & 15) * 8]
                              : (lds_ptr)&sk[0][r * KS + 8 * hh];
    auto kfrag = [&](lds_ptr kt, int i) {  // i = 2*kk + tt
        if constexpr (PG) return *reinterpret_cast<lds_v8>(kt + (i & 1) * 32 * D + (i >> 1) * 256);
        else return *reinterpret_cast<lds_v8>(kt + (i & 1) * 32 * KS + (i >> 1) * 16);
    };
    // V^T operand by two transposing reads: in each 16-lane group, lane j
    // points at key row kb + j/4, dims db + 4 (j % 4) .. +3; lane i then holds
    // keys kb .. kb+3 of dim db + i.  Lane offsets (elements) per dim tile dt:
    const int jg = lane & 15, grp = lane >> 4;
    const int vrow = 4 * hh + (jg >> 2);
    const int vq = 2 * (grp & 1) + ((jg & 3) >> 1);
    int voff[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
        voff[dt] = vrow * D + 32 * (dt ^ ((jg >> 2) & VSW)) + 8 * vq + 4 * (jg & 1);
    // paged: lane i of dim tile dt reads dim 32 dt + i, keys 16 ks + 8 hh .. +7 (page ks)
    const int vdl = lane & 31;
    const lds_ptr v_lane_pg = (lds_ptr)&sv[0][vdl * 16 + 8 * (hh ^ (((vdl >> 2) ^ (vdl >> 3)) & 1))];
    auto vfrag = [&](int buf, int i) {  // i = NDT*ks + dt: keys 16 ks + {4hh..+3, 8+4hh..+3}
        const int dt = i % NDT, ks = i / NDT;
        if constexpr (PG) {
            return *reinterpret_cast<lds_v8>(v_lane_pg + buf * (BN * D) + ks * 16 * D + dt * 512);
        } else {
            const lds_ptr base = (lds_ptr)&sv[buf][0] + voff[dt] + (16 * ks) * D;
            const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)base);
            const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(base + 8 * D));
            const v4 l4 = __builtin_bit_cast(v4, lo), h4 = __builtin_bit_cast(v4, hi);
            return v8{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
        }
    };
    constexpr int PF = 4;

    f32x16 s[2];
    v8 pb[4];  // P^T operand of the tile whose PV is pending
    auto run_pv = [&](int buf) {
        constexpr int NM = 4 * NDT;  // MFMAs: 4 key steps x NDT dim tiles
        v8 vf[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i) vf[i] = vfrag(buf, i);
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            const v8 va = vf[i % PF];
            if (i + PF < NM) vf[i % PF] = vfrag(buf, i + PF);
            o[i % NDT] = Mfma<T>::mma(va, pb[i / NDT], o[i % NDT]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * PF, 0);
#pragma unroll
        for (int i = 0; i < NM - PF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);
    };
    auto run_qk = [&](int buf) {
        constexpr int NM = 2 * (D / 16);  // MFMAs: 2 key halves x D/16 dim steps
        const lds_ptr kt = k_lane + buf * (BN * KS);
        s[0] = f32x16{};
        s[1] = f32x16{};
        v8 kf[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i) kf[i] = kfrag(kt, i);
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            const v8 ka = kf[i % PF];
            if (i + PF < NM) kf[i % PF] = kfrag(kt, i + PF);
            s[i & 1] = Mfma<T>::mma(ka, qr[i >> 1], s[i & 1]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
        for (int i = 0; i < NM - PF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);
    };
    auto phase_softmax = [&](int t, bool masked, unsigned bad) {
        const int k0 = t * BN;
        if (masked) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int kr = PG ? 16 * (e >> 3) + 8 * hh + 4 * ((e >> 2) & 1) + (e & 3)
                                      : 8 * (e >> 2) + 4 * hh + (e & 3);
                    const int key = k0 + 32 * tt + kr;
                    if (key >= Sk || (a.causal && key > q_off + qpos) || ((bad >> ((32 * tt + kr) >> 4)) & 1))
                        s[tt][e] = -INFINITY;
                }
        }
        // exps against the current running max; their sum also tells whether a score
        // outgrew it (see kSumCap), and only then is the max taken and the tile redone
        auto exps = [&]() {
            float ls[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int tt = ks >> 1, i0 = 2 * (ks & 1);
                float p[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    p[j] = fast_exp2(__builtin_fmaf(s[tt][4 * i0 + j], c, -m_run));
                    p[4 + j] = fast_exp2(__builtin_fmaf(s[tt][4 * (i0 + 1) + j], c, -m_run));
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) pb[ks][j] = (T)p[j];
                ls[ks] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            }
            return (ls[0] + ls[1]) + (ls[2] + ls[3]);
        };
        float lt = exps();
        if (__any(!(lt <= kSumCap))) {
            const float mx = wave_max_xor(max32(s[0], s[1]), 32);
            const float m_new = fmaxf(m_run, mx * c);
            const float alpha = fast_exp2(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < D / 32; ++i) o[i] *= alpha;
            m_run = m_new;
            lt = exps();
        }
        l_run += lt;
    };

    issue_unit(0);
    if (nloc >= 1) issue_unit(1);
    __builtin_amdgcn_s_waitcnt(0);  // all counters (Q loads, units 0 and 1)
    barrier();
    // The MFMA phase runs at a raised wave priority so that its MFMA and LDS
    // issues win over the other wave's softmax VALU stream on the same SIMD.
    auto mfma_phase = [&](int t) {
        const bool pv = t >= 1 && tb + t - 1 < w_tiles;
        const bool qk = t < nloc && tb + t < w_tiles;
        __builtin_amdgcn_s_setprio(2);
        if (pv) run_pv(t % NB);
        if (qk) run_qk(t % NB);
        __builtin_amdgcn_s_setprio(0);
    };
    if constexpr (NW == 8) {
        // this wave's loads per unit (K + V): 5 for wave 0 and 4 for the others with the
        // padded contiguous K tile (17 loads); from the pool D / 16 for a lead wave and none
        // for a lag wave
        constexpr int NLP = LPD * ((K_INSTR / NW) + VJ);
        const int nl = PG ? NLP : (wave == 0 ? 3 : 2) + 2;
        // Wait until this wave's loads of unit u are complete while its loads of
        // the next `ahead` units (0, 1 or 2) may still be in flight.
        // vmcnt(n) on gfx9: bits 3:0 and 15:14; expcnt 6:4 = 7; lgkmcnt 11:8 = 15
#define PI_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0F70 | ((n) & 15) | (((n) >> 4) << 14))
        auto wait_unit = [&](int ahead) {
            if (ahead == 2) {
                if (PG) PI_VMCNT(2 * NLP);
                else if (nl == 5) PI_VMCNT(10);
                else PI_VMCNT(8);
            } else if (ahead == 1) {
                if (PG) PI_VMCNT(NLP);
                else if (nl == 5) PI_VMCNT(5);
                else PI_VMCNT(4);
            } else {
                PI_VMCNT(0);
            }
        };
#undef PI_VMCNT
        auto ahead_of = [&](int u) { return min(2, max(0, nloc - u)); };
        // One barrier per tile step t = 0 .. n_tiles.  Lead waves (0-3): the
        // MFMA phase of tile t, then the softmax of tile t; lag waves (4-7): the
        // softmax of tile t-1, then the MFMA phase of tile t; so the two
        // wavefronts of each SIMD alternate phases inside a step.  Each wave
        // issues its loads of unit t+3 in step t (the buffer's previous unit,
        // t-1, was last read in step t-1) and waits for unit t+1 before the
        // barrier.
        if (2 <= nloc) issue_unit(2);
        if (wave < NW / 2) {
            for (int t = 0; t <= nloc; ++t) {
                mfma_phase(t);
                if (t < nloc && tb + t < w_tiles) {
                    const unsigned bd = (bad_units >> (4 * (t % NB))) & 15;
                    phase_softmax(tb + t, tb + t >= t_mask || bd, bd);
                }
                if (t + 3 <= nloc) issue_unit(t + 3);
                if (t < nloc) {
                    wait_unit(ahead_of(t + 1));
                    barrier();
                }
            }
        } else {
            for (int t = 0; t <= nloc; ++t) {
                if (t >= 1 && tb + t - 1 < w_tiles) {
                    const unsigned bd = (bad_units >> (4 * ((t - 1) % NB))) & 15;
                    phase_softmax(tb + t - 1, tb + t - 1 >= t_mask || bd, bd);
                }
                if (t + 3 <= nloc) issue_unit(t + 3);
                mfma_phase(t);
                if (t < nloc) {
                    wait_unit(ahead_of(t + 1));
                    barrier();
                }
            }
        }
    } else {
        // One wavefront per SIMD and two buffers: in step t each wave issues
        // its loads of unit t+1 (the buffer's previous unit, t-1, was last read
        // in step t-1), runs the MFMA phase and the softmax of tile t, and
        // waits for unit t+1 before the barrier.
        for (int t = 0; t <= nloc; ++t) {
            if (t >= 1 && t + 1 <= nloc) issue_unit(t + 1);
            mfma_phase(t);
            if (t < nloc && tb + t < w_tiles) {
                const unsigned bd = (bad_units >> (4 * (t % NB))) & 15;
                phase_softmax(tb + t, tb + t >= t_mask || bd, bd);
            }
            if (t < nloc) {
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
                barrier();
            }
        }
    }

    l_run = wave_sum_xor(l_run, 32);
    if (split) {  // unnormalised partial of this key split
        if (qpos < S) {
            const size_t row = (((size_t)ksp * (gridDim.z / a.ksplit) + b) * S + qpos) * a.hq + head;
            float* po = a.part_o + row * D;
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    f32x4 t = {o[dt][4 * i], o[dt][4 * i + 1], o[dt][4 * i + 2], o[dt][4 * i + 3]};
                    *reinterpret_cast<f32x4*>(po + 32 * dt + 8 * i + 4 * hh) = t;
                }
            if (hh == 0) {
                a.part_ml[2 * row] = m_run;
                a.part_ml[2 * row + 1] = l_run;
            }
        }
    } else if (qpos < S) {
        const float inv = 1.0f / l_run;
        const size_t ro = (((size_t)b * S + qpos) * a.hq + head) * D;
        float* orow = a.out + ro;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f32x4 t = {o[dt][4 * i] * inv, o[dt][4 * i + 1] * inv, o[dt][4 * i + 2] * inv,
                           o[dt][4 * i + 3] * inv};
                if (a.gate) {
                    const f32x4 gt = *reinterpret_cast<const f32x4*>(a.gate + ro + 32 * dt + 8 * i + 4 * hh);
#pragma unroll
                    for (int e = 0; e < 4; ++e) t[e] *= gate_sigmoid(gt[e]);
                }
                *reinterpret_cast<f32x4*>(orow + 32 * dt + 8 * i + 4 * hh) = t;
            }
    }
    }  // query blocks of this workgroup
}

// ---------------------------------------------------------------------------
// prefill_fa256_kernel: head dim 256 with two wavefronts per SIMD.  At 32 query
// rows a wavefront's O and Q^T alone take 192 registers, so prefill_fa_kernel
// runs D = 256 with one wavefront per SIMD, whose MFMA and softmax phases then
// cannot overlap.  Here a wavefront owns 16 query rows on
// v_mfma_f32_16x16x32 (O^T 64 registers, Q^T 32), so the workgroup has 8
// wavefronts (two per SIMD, in opposite phases as in prefill_fa_kernel) and
// covers the same 128 query rows per head set.  Per 64-key tile and wavefront:
//   S^T[64 key x 16 q] = K . Q^T    (4 key blocks x 8 dim steps = 32 MFMAs)
//   O^T[256 x 16 q]   += V^T . P^T  (16 dim blocks x 2 key steps = 32 MFMAs)
// A lane holds query column lane % 16 and keys 16 kb + 4 (lane / 16) + r of
// each key block kb, so the P^T operand of key step j is the lane's own P of
// blocks 2j and 2j+1 (contraction slot 8 g + i is key 32 j + 4 g + i, slot
// 8 g + 4 + i key 32 j + 16 + 4 g + i), and the row max / sum need two
// cross-lane steps.  Units (K of tile u, V of tile u - 1) live in two LDS
// buffers: K rows padded to 544 bytes (two rows apart differ by 2 16-byte
// chunks of banks, so the K reads, 16 rows x 4 chunks per instruction, have no
// bank conflicts; the 528-byte rows of prefill_fa_kernel lost 0.2 of the LDS
// cycles to conflicts here), V rows of 512 bytes whose 16-byte chunks sit at
// chunk ^ 2 (row % 8), so the 16 rows one transposing read touches fall on 8
// distinct bank groups.
// ---------------------------------------------------------------------------
template <typename T>
struct Mfma16;
template <>
struct Mfma16<bf16> {
    static __device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mfma16<f16> {
    static __device__ __forceinline__ f32x4 mma(f16x8 a, f16x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

__device__ __forceinline__ float max16(const f32x4* s) {
    const float a = vmax3(s[0][0], s[0][1], s[0][2]), b = vmax3(s[0][3], s[1][0], s[1][1]);
    const float c = vmax3(s[1][2], s[1][3], s[2][0]), d = vmax3(s[2][1], s[2][2], s[2][3]);
    const float e = vmax3(s[3][0], s[3][1], s[3][2]);
    return vmax3(vmax3(a, b, c), vmax3(d, e, s[3][3]), a);
}

template <typename T, int HPW, bool PG>
__global__ __launch_bounds__(512, 1) void prefill_fa256_kernel(PrefillArgs a) {
    typedef typename Mfma<T>::v8 v8;
    typedef short s4 __attribute__((ext_vector_type(4)));
    constexpr int D = 256, NW = 8, R = 16;  // head dim, wavefronts, query rows per wavefront
    constexpr int RT = NW / HPW;            // row tiles per workgroup
    constexpr int WROWS = R * RT;           // query rows per workgroup (128 / HPW)
    constexpr int NB = 2;                   // unit buffers
    constexpr int NDB = D / 16;             // 16-dim blocks of O^T
    constexpr int KS = D + 16;              // K row stride (elements): 32 bytes of padding
    constexpr int KCH = KS / 8;             // 34 16-byte chunks per K row
    constexpr int K_INSTR = BN * KCH / 64;  // 34 direct loads of 1 KB per K tile
    constexpr int KJ = (K_INSTR + NW - 1) / NW;
    constexpr int V_INSTR = BN * D * 2 / 1024;  // 32 per V tile
    constexpr int VJ = V_INSTR / NW;
    constexpr int VRPI = 1024 / (2 * D);  // V rows per load (2)
    constexpr int VCPR = D / 8;           // 16-byte chunks per V row (32)
    static_assert(WROWS * HPW == 128, "the launch geometry assumes 128 rows per head set");
    __shared__ __attribute__((aligned(1024))) T sk[NB][BN * KS];
    __shared__ __attribute__((aligned(1024))) T sv[NB][BN * D];

    {  // a head that does not exist (modulo map, HPW 1) makes the whole workgroup leave
        const int per_kv = a.group / HPW;
        const int hs0 = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) % HPW;
        if (head_of((int)blockIdx.x / per_kv, ((int)blockIdx.x % per_kv) * HPW + hs0, a.hkv,
                    a.group, a.gqa_mode) >= a.hq)
            return;
    }
    const int nqb = (a.S + WROWS - 1) / WROWS;
    const int by = blockIdx.y;
    const int n_blocks = a.paired && by != nqb - 1 - by ? 2 : 1;
    for (int blk = 0; blk < n_blocks; ++blk) {
    int qb = blk == 0 ? (a.paired ? nqb - 1 - by : (int)gridDim.y - 1 - by) : by;
    if (blk > 0) {  // the previous block's LDS reads are done before new loads land
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }
    int tid = threadIdx.x, bxx = blockIdx.x;
    asm volatile("" : "+v"(tid));
    asm volatile("" : "+s"(bxx), "+s"(qb));
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hs = wave % HPW, rt = wave / HPW;
    const int b = (int)blockIdx.z / a.ksplit, ksp = (int)blockIdx.z % a.ksplit;
    const int S = a.S, Sk = a.Sk, q_off = a.q_off;
    const int per_kv = a.group / HPW;
    const int kvh = bxx / per_kv;
    const int head = head_of(kvh, (bxx % per_kv) * HPW + hs, a.hkv, a.group, a.gqa_mode);
    const int p0 = qb * WROWS + rt * R;
    const int wg_keys = a.causal ? min(Sk, q_off + qb * WROWS + WROWS) : Sk;
    const int n_tiles = (wg_keys + BN - 1) / BN;
    const int pieces = split_pieces(n_tiles, a.ksplit, a.kthr);
    if (ksp >= pieces) continue;  // uniform per workgroup
    const bool split = pieces > 1;
    const int kper = (n_tiles + pieces - 1) / pieces;
    const int tb = min(n_tiles, ksp * kper);
    const int nloc = min(n_tiles, tb + kper) - tb;
    const int w_keys = a.causal ? min(Sk, q_off + p0 + R) : Sk;
    const int w_tiles = p0 < S ? (w_keys + BN - 1) / BN : 0;
    const int t_mask = min(a.causal ? (q_off + p0 + 1) / BN : Sk / BN, Sk / BN);

    const int ln = lane & 15;  // query column of this lane
    const int g = lane >> 4;   // 8-wide contraction slice of the operands
    const int qpos = p0 + ln;

    // Q^T operand: lane holds q[qpos][32 ks + 8 g .. +7]
    v8 qr[D / 32];
    if (PG && a.q_f32) {  // f32 query rows, rounded to T here (RNE)
        const float* qg = reinterpret_cast<const float*>(a.q);
        const bool ok = qpos < S;
        const float* qrow = qg + (((size_t)b * S + (ok ? qpos : 0)) * a.hq + head) * D;
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const f32x4 lo = *reinterpret_cast<const f32x4*>(qrow + 32 * ks + 8 * g);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(qrow + 32 * ks + 8 * g + 4);
            v8 t = {(T)lo[0], (T)lo[1], (T)lo[2], (T)lo[3], (T)hi[0], (T)hi[1], (T)hi[2], (T)hi[3]};
            if (!ok) t = v8{};
            qr[ks] = t;
        }
    } else {
        const T* qg = reinterpret_cast<const T*>(a.q);
        const bool ok = qpos < S;
        const T* qrow = qg + (((size_t)b * S + (ok ? qpos : 0)) * a.hq + head) * D;
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            v8 t = *reinterpret_cast<const v8*>(qrow + 32 * ks + 8 * g);
            if (!ok) t = v8{};
            qr[ks] = t;
        }
    }
    f32x4 o[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -1e30f, l_run = 0.f;

    const size_t tok_stride = (size_t)a.hkv * D;
    const T* kbase = reinterpret_cast<const T*>(a.k) + ((size_t)b * Sk * a.hkv + kvh) * D;
    const T* vbase = reinterpret_cast<const T*>(a.v) + ((size_t)b * Sk * a.hkv + kvh) * D;

    typedef __attribute__((address_space(3))) void lds_void;
    // direct global -> LDS loads from inline assembly (no compiler waits before LDS
    // reads; M0 saved and restored); base and LDS address pinned to scalar registers
    auto dma16 = [](const void* src, lds_void* dst) {
        const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)dst);
        unsigned saved;
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\t"
                     "global_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(src), "s"(lds) : "memory");
    };
    auto dma16s = [](const void* base, unsigned voff, lds_void* dst) {
        const uintptr_t bp = (uintptr_t)base;
        const unsigned blo = __builtin_amdgcn_readfirstlane((unsigned)bp);
        const unsigned bhi = __builtin_amdgcn_readfirstlane((unsigned)(bp >> 32));
        base = (const void*)(((uintptr_t)bhi << 32) | blo);
        const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)dst);
        unsigned saved;
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\t"
                     "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(voff), "s"(base), "s"(lds) : "memory");
    };
    int k_row[KJ], v_row[VJ];
    unsigned k_off[KJ], v_off[VJ];
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
        const int i = wave + NW * j;
        const int L = 64 * (i < K_INSTR ? i : 0) + lane;
        const int row = L / KCH, ch = L - row * KCH;
        k_row[j] = row;
        // the two pad chunks of a row reload its chunks 0 and 1
        k_off[j] = (unsigned)(((size_t)row * tok_stride + 8 * (ch < D / 8 ? ch : ch - D / 8)) * sizeof(T));
    }
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
        const int i = VJ * wave + j;
        const int row = VRPI * i + lane / VCPR;
        const int cc = (lane % VCPR) ^ (2 * (row & 7));
        v_row[j] = row;
        v_off[j] = (unsigned)(((size_t)row * tok_stride + 8 * cc) * sizeof(T));
    }
    auto issue_unit_c = [&](int u) {
        const int buf = u % NB;
        const int k0 = (tb + u) * BN;
        if (k0 + BN <= Sk) {
            const T* kb = kbase + (size_t)k0 * tok_stride;
#pragma unroll
            for (int j = 0; j < KJ; ++j) {
                const int i = wave + NW * j;
                if (i < K_INSTR) dma16s(kb, k_off[j], (lds_void*)&sk[buf][512 * i]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < KJ; ++j) {
                const int i = wave + NW * j;
                if (i < K_INSTR) {
                    const int key = min(k0 + k_row[j], Sk - 1);
                    const T* src = kbase + (size_t)key * tok_stride +
                                   (k_off[j] - (size_t)k_row[j] * tok_stride * sizeof(T)) / sizeof(T);
                    dma16(src, (lds_void*)&sk[buf][512 * i]);
                }
            }
        }
        if (u >= 1) {
            const int v0 = k0 - BN;
            const T* vb = vbase + (size_t)v0 * tok_stride;
            if (v0 + BN <= Sk) {
#pragma unroll
                for (int j = 0; j < VJ; ++j) dma16s(vb, v_off[j], (lds_void*)&sv[buf][512 * (VJ * wave + j)]);
            } else {
#pragma unroll
                for (int j = 0; j < VJ; ++j) {
                    const int key = min(v0 + v_row[j], Sk - 1);
                    const T* src = vbase + (size_t)key * tok_stride +
                                   (v_off[j] - (size_t)v_row[j] * tok_stride * sizeof(T)) / sizeof(T);
                    dma16(src, (lds_void*)&sv[buf][512 * (VJ * wave + j)]);
                }
            }
        }
    };
    // Paged source, page-major unit buffers as in prefill_fa_kernel: K [4 pages][32 chunks]
    // [16 key slots][8] with key k of an odd page in slot k ^ 4, V [4 pages][256 dims][16
    // keys] with dim d's 8-key halves swapped when bit 2 ^ bit 3 of d is set.  Load i moves
    // 1 KB of page i / 8: K chunks 4 (i % 8) .. +3, V dims 32 (i % 8) .. +31; wave w issues
    // slice w of every page (i = w + 8 j, page j).  Page ids as in prefill_fa_kernel: scalar
    // loads, the next unit's read at the start of an issue; a page id outside the pool holds
    // no tokens (page 0 read, keys masked).
    typedef int i32x4_ __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(4))) const int32_t* const_i32p;
    typedef __attribute__((address_space(4))) const i32x4_* const_i32x4p;
    const int last_pg = (Sk - 1) >> 4;
    const unsigned page_bytes_k = (unsigned)(a.hkv * a.kstride), page_bytes_v = (unsigned)(a.hkv * a.vstride);
    const char* kq_pg = a.kpool + (size_t)kvh * a.kstride + 1024 * wave;
    const char* vq_pg = a.vpool + (size_t)kvh * a.vstride + 1024 * wave;
    const int ks_ = lane & 15, vd_ = lane >> 1;
    const unsigned k_lo0 = (unsigned)((lane >> 4) * 256 + 16 * ks_);
    const unsigned k_lo1 = (unsigned)((lane >> 4) * 256 + 16 * (ks_ ^ 4));
    const unsigned v_lo = (unsigned)(vd_ * 32 + 16 * ((lane & 1) ^ (((vd_ >> 2) ^ (vd_ >> 3)) & 1)));
    unsigned koff_prev[4] = {};
    auto load_ids = [&](int u) {
        i32x4_ r = {};
        if constexpr (PG) {
            const int p0_ = (tb + u) * (BN >> 4);
            if (p0_ + 3 <= last_pg) {
                r = *(const_i32x4p)((const_i32p)a.pt + __builtin_amdgcn_readfirstlane(p0_));
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    r[j] = ((const_i32p)a.pt)[__builtin_amdgcn_readfirstlane(min(p0_ + j, last_pg))];
            }
        }
        return r;
    };
    bool ids_ok = true;  // every page id of the workgroup's tiles in the pool (checked once)
    if constexpr (PG) {
        const int pe = min((tb + nloc) * (BN >> 4), last_pg + 1);
        bool bad_l = false;
        for (int pp = tb * (BN >> 4) + lane; pp < pe; pp += 64)
            bad_l |= (unsigned)a.pt[pp] >= (unsigned)a.n_pages;
        ids_ok = !__any(bad_l);
    }
    i32x4_ ids_next = load_ids(0);
    unsigned bad_units = 0;  // 4 bits per unit buffer: the K tile's pages outside the pool
    auto issue_unit_p = [&](int u) {
        const int buf = u % NB;
        const i32x4_ r = ids_next;
        ids_next = load_ids(u + 1);
        if (!ids_ok) {
            unsigned bad = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) bad |= (unsigned)((unsigned)r[j] >= (unsigned)a.n_pages) << j;
            bad_units = (bad_units & ~(15u << (4 * buf))) | (bad << (4 * buf));
        }
        unsigned koff[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            koff[j] = (unsigned)r[j] < (unsigned)a.n_pages ? (unsigned)r[j] : 0u;
            dma16s(kq_pg + (size_t)koff[j] * page_bytes_k, (j & 1) ? k_lo1 : k_lo0,
                   (lds_void*)&sk[buf][512 * (wave + NW * j)]);
        }
        if (u >= 1) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                dma16s(vq_pg + (size_t)koff_prev[j] * page_bytes_v, v_lo, (lds_void*)&sv[buf][512 * (wave + NW * j)]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) koff_prev[j] = koff[j];
    };
    auto issue_unit = [&](int u) {
        if constexpr (PG) issue_unit_p(u);
        else issue_unit_c(u);
    };
    auto barrier = [&]() {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    const float c = a.qk_scale;
    typedef __attribute__((address_space(3))) const T* lds_ptr;
    typedef __attribute__((address_space(3))) const v8* lds_v8;
    typedef __attribute__((address_space(3))) s4* lds_s4;
    // Paged: row rho of key block kb reads key 32 (kb / 2) + 8 (rho / 4) + 4 (kb % 2) +
    // rho % 4, so that the P^T slots 8 g .. 8 g + 7 of key step j (accumulator rows 4 g + r
    // of blocks 2 j, 2 j + 1) are the 8 consecutive keys 32 j + 8 g .. +7: the V^T operand
    // is one 16-byte read of a page's dim row.  Lane offsets (elements) for kb % 2 = 0, 1:
    const int kpar = ln >> 3;  // page parity of this lane's K rows
    const int kpg_base = kpar * 4096 + g * 128 + (8 * ((ln >> 2) & 1) + (ln & 3)) * 8;
    const lds_ptr k_lane_p0 = (lds_ptr)&sk[0][kpg_base + 32 * kpar];
    const lds_ptr k_lane_p1 = (lds_ptr)&sk[0][kpg_base + 32 * (kpar ^ 1)];
    const int vgsw = ((ln >> 2) ^ (ln >> 3)) & 1;
    const lds_ptr v_lane_pg = (lds_ptr)&sv[0][(g >> 1) * 4096 + ln * 16 + 8 * ((g & 1) ^ vgsw)];
    // K operand of key block kb, dim step ks: row 16 kb + ln, elements 32 ks + 8 g .. +7
    const lds_ptr k_lane = (lds_ptr)&sk[0][ln * KS + 8 * g];
    // MFMA i of a QK phase: key block i % 4, dim step i / 4 (four independent accumulators)
    auto kfrag = [&](lds_ptr kt, int i) {
        return *reinterpret_cast<lds_v8>(kt + (i & 3) * 16 * KS + (i >> 2) * 32);
    };
    auto kfrag_p = [&](int buf, int i) {  // paged: key block i % 4, dim step i / 4
        const int kb = i & 3, ks = i >> 2;
        const lds_ptr kl = (kb & 1) ? k_lane_p1 : k_lane_p0;
        return *reinterpret_cast<lds_v8>(kl + buf * (BN * KS) + (kb >> 1) * 8192 + ks * 512);
    };
    // V^T operand of dim block db, key step j by two transposing reads: in the
    // 16-lane group g, lane j' points at key row 32 j + 4 g + j' / 4 (+ 16 for the
    // second read), dims 16 db + 4 (j' % 4) .. +3; lane i then holds 4 keys of dim
    // 16 db + i.  Rows 32 j + 4 g + j'/4 and that + 16 share row % 8.
    const int vrow = 4 * g + (ln >> 2);
    const int vsw = 2 * (vrow & 7);
    auto vfrag = [&](int buf, int i) {  // MFMA i of a PV phase: dim block i % 16, key step i / 16
        const int db = i % NDB, j = i / NDB;
        if constexpr (PG) return *reinterpret_cast<lds_v8>(v_lane_pg + buf * (BN * D) + j * 8192 + db * 256);
        const int ch = (2 * db + ((ln & 3) >> 1)) ^ vsw;
        const lds_ptr base = (lds_ptr)&sv[buf][0] + (32 * j + vrow) * D + 8 * ch + 4 * (ln & 1);
        const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)base);
        const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(base + 16 * D));
        typedef typename Mfma<T>::v4 v4;
        const v4 l4 = __builtin_bit_cast(v4, lo), h4 = __builtin_bit_cast(v4, hi);
        return v8{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
    };
    constexpr int PF = 4;

    f32x4 s[4];
    v8 pb[2];  // P^T operand of the tile whose PV is pending
    auto run_pv = [&](int buf) {
        constexpr int NM = 2 * NDB;  // 32 MFMAs: 16 dim blocks x 2 key steps
        v8 vf[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i) vf[i] = vfrag(buf, i);
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            const v8 va = vf[i % PF];
            if (i + PF < NM) vf[i % PF] = vfrag(buf, i + PF);
            o[i % NDB] = Mfma16<T>::mma(va, pb[i / NDB], o[i % NDB]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * PF, 0);
#pragma unroll
        for (int i = 0; i < NM - PF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);
    };
    auto run_qk = [&](int buf) {
        constexpr int NM = 4 * (D / 32);  // 32 MFMAs: 4 key blocks x 8 dim steps
        const lds_ptr kt = k_lane + buf * (BN * KS);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) s[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto kf_at = [&](int i) {
            if constexpr (PG) return kfrag_p(buf, i);
            else return kfrag(kt, i);
        };
        v8 kf[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i) kf[i] = kf_at(i);
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            const v8 ka = kf[i % PF];
            if (i + PF < NM) kf[i % PF] = kf_at(i + PF);
            s[i & 3] = Mfma16<T>::mma(ka, qr[i >> 2], s[i & 3]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
        for (int i = 0; i < NM - PF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);
    };
    auto phase_softmax = [&](int t, bool masked, unsigned bad) {
        const int k0 = t * BN;
        if (masked) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int kr = PG ? 32 * (kb >> 1) + 8 * g + 4 * (kb & 1) + r : 16 * kb + 4 * g + r;
                    const int key = k0 + kr;
                    if (key >= Sk || (a.causal && key > q_off + qpos) || ((bad >> (kr >> 4)) & 1))
                        s[kb][r] = -INFINITY;
                }
        }
        // exps against the current running max; the max only when their sum says a
        // score outgrew it (see kSumCap)
        auto exps = [&]() {
            float ls[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float p[8];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    p[r] = fast_exp2(__builtin_fmaf(s[2 * j][r], c, -m_run));
                    p[4 + r] = fast_exp2(__builtin_fmaf(s[2 * j + 1][r], c, -m_run));
                }
#pragma unroll
                for (int r = 0; r < 8; ++r) pb[j][r] = (T)p[r];
                ls[j] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            }
            return ls[0] + ls[1];
        };
        float lt = exps();
        if (__any(!(lt <= kSumCap))) {
            float mx = max16(s);
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_run, mx * c);
            const float alpha = fast_exp2(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < NDB; ++i) o[i] *= alpha;
            m_run = m_new;
            lt = exps();
        }
        l_run += lt;
    };
    auto mfma_phase = [&](int t) {
        const bool pv = t >= 1 && tb + t - 1 < w_tiles;
        const bool qk = t < nloc && tb + t < w_tiles;
        __builtin_amdgcn_s_setprio(2);
        if (pv) run_pv(t % NB);
        if (qk) run_qk(t % NB);
        __builtin_amdgcn_s_setprio(0);
    };

    issue_unit(0);
    __builtin_amdgcn_s_waitcnt(0);  // all counters (Q loads, unit 0)
    barrier();
    // One barrier per tile step t = 0 .. nloc.  Lead waves (0-3): the MFMA phase of
    // tile t, then its softmax; lag waves (4-7): the softmax of tile t-1, then the
    // MFMA phase of tile t.  Each wave issues its loads of unit t+1 after its
    // softmax (the buffer's previous unit, t-1, was last read in step t-1) and waits
    // for them before the barrier.
    if (wave < NW / 2) {
        for (int t = 0; t <= nloc; ++t) {
            mfma_phase(t);
            if (t < nloc && tb + t < w_tiles) {
                const unsigned bd = (bad_units >> (4 * (t % NB))) & 15;
                phase_softmax(tb + t, tb + t >= t_mask || bd, bd);
            }
            if (t + 1 <= nloc) issue_unit(t + 1);
            if (t < nloc) {
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
                barrier();
            }
        }
    } else {
        for (int t = 0; t <= nloc; ++t) {
            if (t >= 1 && tb + t - 1 < w_tiles) {
                const unsigned bd = (bad_units >> (4 * ((t - 1) % NB))) & 15;
                phase_softmax(tb + t - 1, tb + t - 1 >= t_mask || bd, bd);
            }
            if (t + 1 <= nloc) issue_unit(t + 1);
            mfma_phase(t);
            if (t < nloc) {
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
                barrier();
            }
        }
    }

    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (split) {  // unnormalised partial of this key split
        if (qpos < S) {
            const size_t row = (((size_t)ksp * (gridDim.z / a.ksplit) + b) * S + qpos) * a.hq + head;
            float* po = a.part_o + row * D;
#pragma unroll
            for (int db = 0; db < NDB; ++db) *reinterpret_cast<f32x4*>(po + 16 * db + 4 * g) = o[db];
            if (g == 0) {
                a.part_ml[2 * row] = m_run;
                a.part_ml[2 * row + 1] = l_run;
            }
        }
    } else if (qpos < S) {
        const float inv = 1.0f / l_run;
        const size_t ro = (((size_t)b * S + qpos) * a.hq + head) * D;
        float* orow = a.out + ro;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            f32x4 t = o[db] * inv;
            if (a.gate) {
                const f32x4 gt = *reinterpret_cast<const f32x4*>(a.gate + ro + 16 * db + 4 * g);
#pragma unroll
                for (int e = 0; e < 4; ++e) t[e] *= gate_sigmoid(gt[e]);
            }
            *reinterpret_cast<f32x4*>(orow + 16 * db + 4 * g) = t;
        }
    }
    }  // query blocks of this workgroup
}

// ---------------------------------------------------------------------------
// prefill_f32_kernel: causal attention of a chunk of queries (f32 rows) over an
// f32 KV pool, read through the sequence's page table (src/model/mod.rs:668
// token loop over :1140-1190 with an f32 cache).  Products keep f32 accuracy
// on the bf16 MFMA by splitting each f32 operand into bf16 hi + lo parts
// (x = hi + lo to 16 significant bits, the exponent range of f32) and summing
// hi.hi + hi.lo + lo.hi: three v_mfma_f32_16x16x32_bf16 per block.
//
// A workgroup of 4 wavefronts covers 64 query rows of one query head; wave w
// owns rows 16 w .. 16 w + 15.  Per 32-key tile (two pool pages):
//   S^T[32 key x 16 q] = K . Q^T   (lane: query column c = lane % 16, keys 4 g + r)
//   O^T[D x 16 q]     += V^T . P^T (P^T's contraction order matches the lane's keys)
// K is staged in LDS as [key][dim] hi / lo rows, V as [dim][key] (the pool's V
// block is already dim-major); the next tile's raw f32 pages are loaded into
// registers while the current tile computes.
// ---------------------------------------------------------------------------
struct PrefillF32Args {
    const float* q;         // [n_tok][hq][D], normalised and rotated
    const float* kpool;     // f32 pool K blocks [D/4][16][4] of (page, kv head) i at kpool + i kstride
    const float* vpool;     // f32 pool V blocks [D][16] at vpool + i vstride
    size_t kstride, vstride;  // bytes
    const int32_t* pt;      // the sequence's page-table row
    float* out;             // [n_tok][hq][D]
    const float* gate;      // optional [n_tok][hq][D]: out *= sigmoid(gate)
    int n_tok, q_off, max_pages, n_pages, hq, hkv, group, gqa_mode;
    float qk_scale;         // scale * log2(e)
};

template <int D>
__global__ __launch_bounds__(256) void prefill_f32_kernel(PrefillF32Args a) {
    constexpr int TK = 32;          // keys per tile (two pages)
    // Row strides (bf16) chosen so that the 16-row x 4-chunk operand reads and the staging
    // writes fall on distinct LDS banks: K rows of D + 16, V^T rows of 40 (80 bytes).
    constexpr int KST = D + 16;     // K row stride (bf16)
    constexpr int VST = TK + 8;     // V^T row stride (bf16)
    constexpr int NF = 2 * TK * D / 4 / 256;  // float4 loads per thread per tile (K and V)
    constexpr int NKS = D / 32;     // 32-dim steps of Q.K
    constexpr int NDB = D / 16;     // 16-dim blocks of O^T
    __shared__ __attribute__((aligned(16))) bf16 skh[TK * KST], skl[TK * KST];
    __shared__ __attribute__((aligned(16))) bf16 svh[D * VST], svl[D * VST];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int qb = gridDim.x - 1 - blockIdx.x;  // heaviest (latest) query blocks first
    const int head = blockIdx.y;
    const int kvh = a.gqa_mode == 0 ? head % a.hkv : head / a.group;
    const int L = a.q_off + a.n_tok;            // keys of the sequence after this chunk
    const int p0 = qb * 64 + 16 * wave;         // this wave's first query row
    const int wg_keys = min(L, a.q_off + qb * 64 + 64);
    const int n_tiles = (wg_keys + TK - 1) / TK;
    const int w_keys = min(L, a.q_off + p0 + 16);
    const int w_tiles = p0 < a.n_tok ? (w_keys + TK - 1) / TK : 0;
    const int qpos = p0 + c;

    // Q^T operand (B of K.Q^T): lane holds q[qpos][32 ks + 8 g .. +7] as hi / lo
    bf16x8 qh[NKS], ql[NKS];
    {
        const bool ok = qpos < a.n_tok;
        const float* qr = a.q + ((size_t)(ok ? qpos : 0) * a.hq + head) * D;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            f32x4 x0 = *reinterpret_cast<const f32x4*>(qr + 32 * ks + 8 * g);
            f32x4 x1 = *reinterpret_cast<const f32x4*>(qr + 32 * ks + 8 * g + 4);
            if (!ok) x0 = x1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = j < 4 ? x0[j] : x1[j - 4];
                const bf16 h = to_bf16(x);
                qh[ks][j] = h;
                ql[ks][j] = to_bf16(x - (float)h);
            }
        }
    }
    f32x4 o[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -1e30f, l_run = 0.f;

    // Tile loads: float4 i of a tile (i = tid + 256 j) is K (i < 8 D) or V, of
    // page i / (4 D) % 2; within a page block both are a linear copy.
    f32x4 pre[NF];
    auto load_tile = [&](int t) {
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const int i = tid + 256 * j;
            const bool isv = i >= 8 * D;
            const int ii = isv ? i - 8 * D : i;
            const int half = ii / (4 * D), ci = ii % (4 * D);
            const int lp = 2 * t + half;
            const int pid = lp < a.max_pages ? a.pt[lp] : -1;
            const bool ok = lp * 16 < L && pid >= 0 && pid < a.n_pages;
            const size_t bi = (size_t)(ok ? pid : 0) * a.hkv + kvh;
            const float* base = reinterpret_cast<const float*>(
                isv ? reinterpret_cast<const char*>(a.vpool) + bi * a.vstride
                    : reinterpret_cast<const char*>(a.kpool) + bi * a.kstride);
            pre[j] = ok ? *reinterpret_cast<const f32x4*>(base + 4 * ci) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto stage_tile = [&]() {
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const int i = tid + 256 * j;
            const bool isv = i >= 8 * D;
            const int ii = isv ? i - 8 * D : i;
            const int half = ii / (4 * D), ci = ii % (4 * D);
            bf16x4 h, l;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                h[e] = to_bf16(pre[j][e]);
                l[e] = to_bf16(pre[j][e] - (float)h[e]);
            }
            if (!isv) {  // K block [D/4][16][4]: dims 4 (ci / 16) .. +3 of token ci % 16
                const int off = (16 * half + ci % 16) * KST + 4 * (ci / 16);
                *reinterpret_cast<bf16x4*>(skh + off) = h;
                *reinterpret_cast<bf16x4*>(skl + off) = l;
            } else {     // V block [D][16]: tokens 4 (ci % 4) .. +3 of dim ci / 4
                const int off = (ci / 4) * VST + 16 * half + 4 * (ci % 4);
                *reinterpret_cast<bf16x4*>(svh + off) = h;
                *reinterpret_cast<bf16x4*>(svl + off) = l;
            }
        }
    };
    auto mma = [](bf16x8 x, bf16x8 y, f32x4 acc) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y, acc, 0, 0, 0);
    };
    const float cs = a.qk_scale;
    load_tile(0);
    for (int t = 0; t < n_tiles; ++t) {
        __syncthreads();  // the previous tile's LDS reads are done
        stage_tile();
        if (t + 1 < n_tiles) load_tile(t + 1);
        __syncthreads();
        if (t >= w_tiles) continue;
        // S^T for keys 16 kb + 4 g + r
        f32x4 st[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const int off = (16 * kb + c) * KST + 32 * ks + 8 * g;
                const bf16x8 kh = *reinterpret_cast<const bf16x8*>(skh + off);
                const bf16x8 kl = *reinterpret_cast<const bf16x8*>(skl + off);
                acc = mma(kh, qh[ks], acc);
                acc = mma(kh, ql[ks], acc);
                acc = mma(kl, qh[ks], acc);
            }
            st[kb] = acc;
        }
        const int k0 = t * TK;
        if (k0 + TK > a.q_off + p0 || k0 + TK > L) {  // the tile reaches past a row's last key
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = k0 + 16 * kb + 4 * g + r;
                    if (key >= L || key > a.q_off + qpos) st[kb][r] = -INFINITY;
                }
        }
        float mx = fmaxf(fmaxf(fmaxf(st[0][0], st[0][1]), fmaxf(st[0][2], st[0][3])),
                         fmaxf(fmaxf(st[1][0], st[1][1]), fmaxf(st[1][2], st[1][3])));
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx * cs);
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < NDB; ++i) o[i] *= alpha;
        // P^T operand: contraction slot 8 g + j is key 16 (j / 4) + 4 g + j % 4
        bf16x8 ph, pl;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float p = fast_exp2(__builtin_fmaf(st[j >> 2][j & 3], cs, -m_new));
            l_run += p;
            const bf16 h = to_bf16(p);
            ph[j] = h;
            pl[j] = to_bf16(p - (float)h);
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const int off = (16 * db + c) * VST + 4 * g;
            const bf16x4 h0 = *reinterpret_cast<const bf16x4*>(svh + off);
            const bf16x4 h1 = *reinterpret_cast<const bf16x4*>(svh + off + 16);
            const bf16x4 l0 = *reinterpret_cast<const bf16x4*>(svl + off);
            const bf16x4 l1 = *reinterpret_cast<const bf16x4*>(svl + off + 16);
            const bf16x8 vh = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
            const bf16x8 vl = {l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
            o[db] = mma(vh, ph, o[db]);
            o[db] = mma(vh, pl, o[db]);
            o[db] = mma(vl, ph, o[db]);
        }
    }
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (qpos >= a.n_tok) return;
    const float inv = 1.0f / l_run;
    const size_t ro = ((size_t)qpos * a.hq + head) * D;
    float* orow = a.out + ro;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
        f32x4 t = o[db] * inv;
        if (a.gate) {
            const f32x4 gt = *reinterpret_cast<const f32x4*>(a.gate + ro + 16 * db + 4 * g);
#pragma unroll
            for (int e = 0; e < 4; ++e) t[e] *= gate_sigmoid(gt[e]);
        }
        *reinterpret_cast<f32x4*>(orow + 16 * db + 4 * g) = t;
    }
}

// The key splits of a prefill launch combined per (batch, query row, head): the
// log-sum-exp merge of the splits' (max, sum) in log2 units and their O.  Each thread
// takes 4 consecutive values of a row (D / 4 threads a row) in MR rows, and requests every
// split's (max, sum) and O and the gate of all of them before it uses any: one memory round
// trip a thread with 16-byte loads, and few enough workgroups that they all fit at once.
// Rows of query positions below q0 (blocks that were not split) are already written; the
// launch starts at row `first`.
template <int D>
constexpr int merge_rows() { return D == 256 ? 1 : 2; }  // MR: rows per thread
template <int D, int KS>
__global__ __launch_bounds__(256) void prefill_merge_kernel(const float* __restrict__ part_o,
                                                            const float* __restrict__ part_ml,
                                                            float* __restrict__ out, long long rows,
                                                            const float* __restrict__ gate,
                                                            long long first, int S, int hq, int q0,
                                                            int kthr, int wrows, int q_off, int Sk,
                                                            int causal) {
    constexpr int LPR = D / 4, RPP = 256 / LPR, MR = merge_rows<D>();
    typedef float f2 __attribute__((ext_vector_type(2)));
    const int c = 4 * ((int)threadIdx.x % LPR);
    long long rw[MR];
    bool live[MR];
    int pcs[MR];
    f2 ml[MR][KS];
    f32x4 o[MR][KS], gt[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        rw[m] = first + ((long long)blockIdx.x * MR + m) * RPP + (int)threadIdx.x / LPR;
        const int qpos = (int)((rw[m] / hq) % S);
        const int keys = causal ? min(Sk, q_off + (qpos / wrows) * wrows + wrows) : Sk;
        pcs[m] = split_pieces((keys + BN - 1) / BN, KS, kthr);  // the row's block's pieces
        live[m] = rw[m] < rows && qpos >= q0 && pcs[m] > 1;
        const long long rl = live[m] ? rw[m] : first;  // a row that exists: loads stay unconditional
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const long long r = (k < pcs[m] ? k : 0) * rows + rl;  // slots past the pieces: weight 0
            ml[m][k] = *reinterpret_cast<const f2*>(part_ml + 2 * r);
            o[m][k] = *reinterpret_cast<const f32x4*>(part_o + r * D + c);
        }
        if (gate) gt[m] = *reinterpret_cast<const f32x4*>(gate + rl * D + c);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float M = ml[m][0][0];
#pragma unroll
        for (int k = 1; k < KS; ++k) M = fmaxf(M, ml[m][k][0]);
        float L = 0.f;
        f32x4 acc = {};
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const float w = k < pcs[m] ? fast_exp2(ml[m][k][0] - M) : 0.f;
            L += w * ml[m][k][1];
            acc += w * o[m][k];
        }
        acc *= 1.0f / L;
        if (gate) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] *= gate_sigmoid(gt[m][e]);
        }
        if (live[m]) *reinterpret_cast<f32x4*>(out + rw[m] * D + c) = acc;
    }
}

}  // namespace

namespace {
// Head dim 256 runs prefill_fa256_kernel (two wavefronts per SIMD); PI_PREFILL_FA256=0
// selects the one-wavefront-per-SIMD prefill_fa_kernel<., ., 256> instead (read per call).
bool use_fa256() {
    const char* e = std::getenv("PI_PREFILL_FA256");
    return !(e && e[0] == '0');
}

template <int D>
void launch_d(const PrefillArgs& a, int hpw, int n_kv_heads, int seq_len, int batch, bool bf,
              hipStream_t s) {
    constexpr int NW = PrefillCfg<D>::NW;
    // x = workgroup's head set (fastest), y = query block (reversed in the
    // kernel so the heaviest blocks go first); with x = KV head and
    // round-robin dispatch over the 8 XCDs, a KV head's K/V stays in one L2.
    const int rows = ROWS * NW / hpw;
    const int nqb = (seq_len + rows - 1) / rows;
    const dim3 grid(n_kv_heads * (a.group / hpw), a.paired ? (nqb + 1) / 2 : nqb, batch * a.ksplit);
    const dim3 block(64 * NW);
    if constexpr (D == 256) {
        if (use_fa256()) {  // same grid: 128 / hpw query rows per workgroup either way
            const dim3 block8(512);
            switch (hpw) {
                case 4:
                    if (bf) hipLaunchKernelGGL((prefill_fa256_kernel<bf16, 4, false>), grid, block8, 0, s, a);
                    else hipLaunchKernelGGL((prefill_fa256_kernel<f16, 4, false>), grid, block8, 0, s, a);
                    break;
                case 2:
                    if (bf) hipLaunchKernelGGL((prefill_fa256_kernel<bf16, 2, false>), grid, block8, 0, s, a);
                    else hipLaunchKernelGGL((prefill_fa256_kernel<f16, 2, false>), grid, block8, 0, s, a);
                    break;
                default:
                    if (bf) hipLaunchKernelGGL((prefill_fa256_kernel<bf16, 1, false>), grid, block8, 0, s, a);
                    else hipLaunchKernelGGL((prefill_fa256_kernel<f16, 1, false>), grid, block8, 0, s, a);
            }
            return;
        }
    }
    switch (hpw) {
        case 4:
            if (bf) hipLaunchKernelGGL((prefill_fa_kernel<bf16, 4, D, false>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((prefill_fa_kernel<f16, 4, D, false>), grid, block, 0, s, a);
            break;
        case 2:
            if (bf) hipLaunchKernelGGL((prefill_fa_kernel<bf16, 2, D, false>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((prefill_fa_kernel<f16, 2, D, false>), grid, block, 0, s, a);
            break;
        default:
            if (bf) hipLaunchKernelGGL((prefill_fa_kernel<bf16, 1, D, false>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((prefill_fa_kernel<f16, 1, D, false>), grid, block, 0, s, a);
    }
}
}  // namespace

hipError_t launch_prefill_f32(const KvGeom& g, const float* q, const int32_t* page_table,
                              int32_t max_pages, int32_t q_off, int32_t n_tok, int32_t n_q_heads,
                              int32_t gqa_mode, float scale, float* out, hipStream_t s,
                              const float* gate) {
    if (g.dtype != 0 || q_off < 0 || n_tok < 1 || max_pages < 1) return hipErrorInvalidValue;
    const bool multiple = n_q_heads % g.n_kv_heads == 0;
    if (!multiple && gqa_mode != 0) return hipErrorInvalidValue;
    PrefillF32Args a;
    a.q = q;
    a.kpool = reinterpret_cast<const float*>(g.k);
    a.vpool = reinterpret_cast<const float*>(g.v);
    a.kstride = g.kstride;
    a.vstride = g.vstride;
    a.pt = page_table;
    a.out = out;
    a.gate = gate;
    a.n_tok = n_tok;
    a.q_off = q_off;
    a.max_pages = max_pages;
    a.n_pages = g.n_pages;
    a.hq = n_q_heads;
    a.hkv = g.n_kv_heads;
    a.group = (n_q_heads + g.n_kv_heads - 1) / g.n_kv_heads;
    a.gqa_mode = gqa_mode;
    a.qk_scale = scale * kLog2e;
    const dim3 grid((unsigned)((n_tok + 63) / 64), (unsigned)n_q_heads);
    switch (g.head_dim) {
        case 64: hipLaunchKernelGGL(prefill_f32_kernel<64>, grid, dim3(256), 0, s, a); break;
        case 128: hipLaunchKernelGGL(prefill_f32_kernel<128>, grid, dim3(256), 0, s, a); break;
        case 256: hipLaunchKernelGGL(prefill_f32_kernel<256>, grid, dim3(256), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

namespace {
int cu_count() {
    static int n_cu = -1;
    if (n_cu < 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            v = 0;
        n_cu = v;
    }
    return n_cu;
}

struct PrefillSched {
    int hpw, paired, ksplit;
    bool forced;  // ksplit from PI_PREFILL_KSPLIT
};

// The schedule of a launch.  Causal launches whose pairs of query blocks fill every CU
// once or more pair them (equal work per workgroup).  Otherwise, a launch with fewer
// workgroups than CUs may split a workgroup's keys over up to 4 workgroups (more CUs
// busy, one merge launch after); ksplit is the number of partial slots the workspace
// holds, split_plan picks the pieces.  PI_PREFILL_PAIRED=0 / 1 and PI_PREFILL_KSPLIT=n
// force either choice.
PrefillSched prefill_sched(int batch, int seq_len, int n_q_heads, int n_kv_heads, int head_dim,
                           int causal) {
    PrefillSched sc;
    const bool multiple = n_q_heads % n_kv_heads == 0;
    const int group = (n_q_heads + n_kv_heads - 1) / n_kv_heads;
    sc.hpw = !multiple ? 1 : group % 4 == 0 ? 4 : (group % 2 == 0 ? 2 : 1);
    const int nw = head_dim == 256 ? PrefillCfg<256>::NW : PrefillCfg<128>::NW;
    const int rows = ROWS * nw / sc.hpw;
    const long long wgs = (long long)n_kv_heads * (group / sc.hpw) * batch * ((seq_len + rows - 1) / rows);
    const long long pairs = (long long)n_kv_heads * (group / sc.hpw) * batch *
                            (((seq_len + rows - 1) / rows + 1) / 2);
    const int n_cu = cu_count();
    sc.paired = causal && n_cu > 0 && pairs >= n_cu;
    const char* env_p = std::getenv("PI_PREFILL_PAIRED");  // read per call, as is PI_PREFILL_KSPLIT
    if (env_p && causal) sc.paired = env_p[0] == '1';
    sc.ksplit = 1;
    sc.forced = false;
    if (!sc.paired && n_cu > 0 && wgs < n_cu) sc.ksplit = (int)std::min<long long>(4, 2 * (n_cu / wgs));
    const char* env_k = std::getenv("PI_PREFILL_KSPLIT");
    if (env_k && !sc.paired) {
        sc.ksplit = std::max(1, std::min(4, std::atoi(env_k)));
        sc.forced = true;
    }
    return sc;
}

// The key split of a launch with a.ksplit > 1 slots, wrows query rows per block and hsets
// workgroups per query block (head sets x batch).  Picks the piece size kthr: the smallest
// for which every block fits the slots and all pieces together fit the CUs once (one
// workgroup a CU: the longest piece sets the launch's time), so short causal blocks run
// whole and long ones in two to four pieces; forced, kthr = ceil(most tiles / ksplit).
// Sets a.kthr and a.ksplit (the most pieces of a block; 1: no split); returns the first
// query row of a split block (S when none is: nothing to merge).
int split_plan(PrefillArgs& a, int wrows, long long hsets, bool forced) {
    const int nqb = (a.S + wrows - 1) / wrows;
    auto tiles = [&](int qb) {
        const int keys = a.causal ? std::min(a.Sk, a.q_off + qb * wrows + wrows) : a.Sk;
        return (keys + BN - 1) / BN;
    };
    const int most = tiles(nqb - 1);  // tiles grow with the block (causal) or are equal
    int p = (most + a.ksplit - 1) / a.ksplit;
    if (!forced) {
        const long long n_cu = cu_count();
        for (; p < most; ++p) {
            long long tot = 0;
            for (int qb = 0; qb < nqb; ++qb) tot += (tiles(qb) + p - 1) / p;
            if (tot * hsets <= n_cu) break;
        }
    }
    a.kthr = std::max(1, p);
    a.ksplit = std::min(a.ksplit, (most + a.kthr - 1) / a.kthr);
    if (a.ksplit <= 1) {
        a.ksplit = 1;
        a.kthr = 0;
        return a.S;
    }
    for (int qb = 0; qb < nqb; ++qb)
        if (tiles(qb) > a.kthr) return qb * wrows;
    return a.S;
}

// The merge of the split blocks' rows (batch, query row >= q0, head) into out.
hipError_t launch_merge(int D, const PrefillArgs& a, int batch, int q0, int wrows, float* out,
                        hipStream_t s) {
    if (q0 >= a.S) return hipSuccess;
    const long long rows = (long long)batch * a.S * a.hq;
    const long long first = batch == 1 ? (long long)q0 * a.hq : 0;
    const long long per_wg = (D == 256 ? merge_rows<256>() : D == 128 ? merge_rows<128>() : merge_rows<64>()) *
                             (256 / (D / 4));
    const dim3 grid((unsigned)((rows - first + per_wg - 1) / per_wg));
#define PI_MERGE_K(DD, KK)                                                                         \
    hipLaunchKernelGGL((prefill_merge_kernel<DD, KK>), grid, dim3(256), 0, s, a.part_o, a.part_ml, out, \
                       rows, a.gate, first, a.S, a.hq, q0, a.kthr, wrows, a.q_off, a.Sk, a.causal)
#define PI_MERGE(DD)                                                                               \
    switch (a.ksplit) {                                                                            \
        case 2: PI_MERGE_K(DD, 2); break;                                                          \
        case 3: PI_MERGE_K(DD, 3); break;                                                          \
        default: PI_MERGE_K(DD, 4);                                                                \
    }
    if (a.ksplit < 2 || a.ksplit > 4) return hipErrorInvalidValue;
    if (D == 256) PI_MERGE(256)
    else if (D == 128) PI_MERGE(128)
    else PI_MERGE(64)
#undef PI_MERGE
#undef PI_MERGE_K
    return hipGetLastError();
}
}  // namespace

size_t prefill_ws_floats(int32_t batch, int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads,
                         int32_t head_dim, int32_t causal) {
    if (batch <= 0 || seq_len <= 0 || n_q_heads <= 0 || n_kv_heads <= 0) return 0;
    const PrefillSched sc = prefill_sched(batch, seq_len, n_q_heads, n_kv_heads, head_dim, causal);
    if (sc.ksplit <= 1) return 0;
    return (size_t)sc.ksplit * batch * seq_len * n_q_heads * (head_dim + 2);
}

hipError_t launch_prefill(const void* q, const void* k, const void* v, int32_t dtype,
                          int32_t batch, int32_t seq_len, int32_t n_keys, int32_t q_off,
                          int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t causal,
                          int32_t gqa_mode, float scale, float* out, float* ws, size_t ws_floats,
                          hipStream_t s, const float* gate) {
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return hipErrorInvalidValue;
    if (q_off < 0 || n_keys < 1 || (causal && q_off + seq_len > n_keys)) return hipErrorInvalidValue;
    PrefillArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.S = seq_len;
    a.Sk = n_keys;
    a.q_off = q_off;
    a.hq = n_q_heads;
    a.hkv = n_kv_heads;
    const bool multiple = n_q_heads % n_kv_heads == 0;
    if (!multiple && gqa_mode != 0) return hipErrorInvalidValue;
    // query heads per KV head (modulo map: up to ceil(Hq / Hkv), the last ones may not exist)
    a.group = (n_q_heads + n_kv_heads - 1) / n_kv_heads;
    a.causal = causal;
    a.gqa_mode = gqa_mode;
    a.qk_scale = scale * kLog2e;
    const bool bf = dtype == 2;
    const PrefillSched sc = prefill_sched(batch, seq_len, n_q_heads, n_kv_heads, head_dim, causal);
    a.paired = sc.paired;
    a.ksplit = 1;
    a.kthr = 0;
    a.part_o = a.part_ml = nullptr;
    a.gate = gate;
    const size_t rows = (size_t)batch * seq_len * n_q_heads;
    int q0 = seq_len;
    const int wrows = ROWS * (head_dim == 256 ? PrefillCfg<256>::NW : PrefillCfg<128>::NW) / sc.hpw;
    if (sc.ksplit > 1 && ws && ws_floats >= (size_t)sc.ksplit * rows * (head_dim + 2)) {
        a.ksplit = sc.ksplit;
        a.part_o = ws;
        a.part_ml = ws + (size_t)sc.ksplit * rows * head_dim;
        q0 = split_plan(a, wrows, (long long)n_kv_heads * (a.group / sc.hpw) * batch, sc.forced);
    }
    if (head_dim == 64) launch_d<64>(a, sc.hpw, n_kv_heads, seq_len, batch, bf, s);
    else if (head_dim == 128) launch_d<128>(a, sc.hpw, n_kv_heads, seq_len, batch, bf, s);
    else launch_d<256>(a, sc.hpw, n_kv_heads, seq_len, batch, bf, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.ksplit == 1) return e;
    return launch_merge(head_dim, a, batch, q0, wrows, out, s);
}

hipError_t launch_prefill_pool(const KvGeom& g, const void* q, int32_t q_f32, const int32_t* page_table,
                               int32_t q_off, int32_t n_tok, int32_t n_q_heads, int32_t gqa_mode,
                               float scale, float* out, float* ws, size_t ws_floats, hipStream_t s,
                               const float* gate) {
    const int D = g.head_dim;
    if (g.dtype != 1 || (D != 64 && D != 128 && D != 256) || q_off < 0 || n_tok < 1) return hipErrorInvalidValue;
    if ((uint64_t)g.n_kv_heads * std::max(g.kstride, g.vstride) >= (1ull << 32)) return hipErrorInvalidValue;
    const bool multiple = n_q_heads % g.n_kv_heads == 0;
    if (!multiple && gqa_mode != 0) return hipErrorInvalidValue;
    PrefillArgs a;
    a.q = q;
    a.k = a.v = nullptr;
    a.out = out;
    a.S = n_tok;
    a.Sk = q_off + n_tok;
    a.q_off = q_off;
    a.hq = n_q_heads;
    a.hkv = g.n_kv_heads;
    a.group = (n_q_heads + g.n_kv_heads - 1) / g.n_kv_heads;
    a.causal = 1;
    a.gqa_mode = gqa_mode;
    a.qk_scale = scale * kLog2e;
    a.gate = gate;
    a.pt = page_table;
    a.kpool = static_cast<const char*>(g.k);
    a.vpool = static_cast<const char*>(g.v);
    a.kstride = g.kstride;
    a.vstride = g.vstride;
    a.n_pages = g.n_pages;
    a.q_f32 = q_f32;
    const PrefillSched sc = prefill_sched(1, n_tok, n_q_heads, g.n_kv_heads, D, 1);
    a.paired = sc.paired;
    a.ksplit = 1;
    a.kthr = 0;
    a.part_o = a.part_ml = nullptr;
    const size_t rows = (size_t)n_tok * n_q_heads;
    // 256 / hpw query rows per workgroup (128 / hpw at D = 256), 8 wavefronts either way
    const int wrows = ROWS * (D == 256 ? PrefillCfg<256>::NW : PrefillCfg<128>::NW) / sc.hpw;
    int q0 = n_tok;
    if (sc.ksplit > 1 && ws && ws_floats >= (size_t)sc.ksplit * rows * (D + 2)) {
        a.ksplit = sc.ksplit;
        a.part_o = ws;
        a.part_ml = ws + (size_t)sc.ksplit * rows * D;
        q0 = split_plan(a, wrows, (long long)g.n_kv_heads * (a.group / sc.hpw), sc.forced);
    }
    const int nqb = (n_tok + wrows - 1) / wrows;
    const dim3 grid(g.n_kv_heads * (a.group / sc.hpw), a.paired ? (nqb + 1) / 2 : nqb, a.ksplit);
    const dim3 block(512);
#define PI_PAGED(DD)                                                                                 \
    switch (sc.hpw) {                                                                                \
        case 4: hipLaunchKernelGGL((prefill_fa_kernel<f16, 4, DD, true>), grid, block, 0, s, a); break; \
        case 2: hipLaunchKernelGGL((prefill_fa_kernel<f16, 2, DD, true>), grid, block, 0, s, a); break; \
        default: hipLaunchKernelGGL((prefill_fa_kernel<f16, 1, DD, true>), grid, block, 0, s, a);      \
    }
    if (D == 256) {
        switch (sc.hpw) {
            case 4: hipLaunchKernelGGL((prefill_fa256_kernel<f16, 4, true>), grid, block, 0, s, a); break;
            case 2: hipLaunchKernelGGL((prefill_fa256_kernel<f16, 2, true>), grid, block, 0, s, a); break;
            default: hipLaunchKernelGGL((prefill_fa256_kernel<f16, 1, true>), grid, block, 0, s, a);
        }
    } else if (D == 128) {
        PI_PAGED(128)
    } else {
        PI_PAGED(64)
    }
#undef PI_PAGED
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.ksplit == 1) return e;
    return launch_merge(D, a, 1, q0, wrows, out, s);
}

}  // namespace pi
