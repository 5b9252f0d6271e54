// qf_spec_attn.hip — split-KV, GQA-packed verification attention for MI355X (gfx950).
//
// Causal attention for a uniform speculative-decode batch (every request has q_len query tokens)
// over a paged bf16 KV cache; the C ABI is declared in include/qf_spec_attn.h.  Same decomposition
// as the reference (plugin/qwen_fastpath/spec_attn.py:1-10): the cached prefix, which every query of a
// request sees in full, is split across workgroups that stream each kv head once for all the
// q_len * G query rows sharing it; a second kernel attends this step's q_len positions causally and
// merges everything by log-sum-exp.  The kernels themselves are designed for CDNA4:
//
//   prefix kernel, one 256-thread workgroup per (split, request, kv head); the last active split also
//   takes this step's q_len in-flight positions, masked causally per query row:
//   * K and V rows of a 32-position stage are copied global -> LDS with 16-byte direct-to-LDS loads
//     (no VGPR staging), 16-byte pieces XOR-swizzled per row so that the MFMA fragment reads below
//     are free of bank conflicts; a ring of kRing stages keeps kRing - 1 stages in flight while a
//     stage is computed, with one barrier per stage.
//   * Wavefront w takes key tile w & 1 (16 of the stage's 32 positions) and d half w >> 1.
//   * S^T = K . Q^T on v_mfma_f32_16x16x32_bf16 with K as the A operand (16 positions x 32 d) and the
//     packed query rows as B (16 rows), so each lane's accumulator holds 4 positions of ONE row: the
//     online softmax needs only two cross-lane steps per row, and the lane's 4 probabilities are
//     already its B fragment of the next product.
//   * O^T = V^T . P^T on v_mfma_f32_16x16x16_bf16 over the tile's 16 positions and the wavefront's
//     half of the head dimension; each V^T fragment is one transposing LDS read (ds_read_b64_tr_b16)
//     of the row-major V rows.
//   * The two key tiles keep separate softmax states (the two wavefronts of a d half compute the same
//     scores), merged once per split through LDS; wavefronts never exchange state inside the loop.
//   combine kernel, one 256-thread workgroup per (token, head, 64 d values): the row's split partials
//   are merged by log-sum-exp in thread groups, then the groups through LDS.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <unordered_set>

#include "qf_spec_attn.h"

namespace qfa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef const void __attribute__((address_space(1)))* gptr_t;
typedef void __attribute__((address_space(3)))* lptr_t;

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kKeyBlock = QF_SPEC_ATTN_KEY_BLOCK;  // positions per stage
constexpr int kMaxRows = QF_SPEC_ATTN_MAX_ROWS;
constexpr int kTablePages = 1024;  // block-table entries a prefix workgroup holds in LDS at once
constexpr float kLog2e = 1.4426950408889634f;
constexpr size_t kMaxDynLds = 160 * 1024 - 8 * 1024;  // gfx950 LDS per workgroup, less the static arrays
constexpr size_t kDefaultLds = 64 * 1024;

struct AttnArgs {
  const uint16_t* q;
  int64_t sq_t, sq_h;
  const uint16_t* kc;
  int64_t sk_b, sk_t, sk_h;
  const uint16_t* vc;
  int64_t sv_b, sv_t, sv_h;
  const int32_t* bt;
  int64_t sbt;
  const int32_t* seq_lens;
  uint16_t* out;
  int64_t so_t, so_h;
  float* o_part;    // [B][HKV][S][R][D]
  float* lse_part;  // [B][HKV][S][R]
  int B, Q, H, HKV, G, R, page, splits, min_chunk;
  float qk_scale;  // softmax scale * log2(e): scores are kept in base 2
};

// Positions per prefix split (the reference's split arithmetic, spec_attn.py:38-40, with this
// kernel's key block): both kernels derive it from the sequence length alone.
__device__ __forceinline__ int split_chunk(int prefix, int splits, int min_chunk) {
  int c = (prefix + splits - 1) / splits;
  c = c > min_chunk ? c : min_chunk;
  return (c + kKeyBlock - 1) / kKeyBlock * kKeyBlock;
}

// Workgroup barrier for the copy ring.  Each wavefront has already waited for its own copies of the
// stage (wait_vmcnt); no release fence is used, because at workgroup scope it would also wait for
// the copies of later stages, which are LDS writes still in flight.  The acquire fence keeps the
// stage's LDS reads (and the next copies into the ring) after the barrier.
__device__ __forceinline__ void ring_barrier() {
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// s_waitcnt with vmcnt = n (0..63) and the other counters unconstrained.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// 32-bit LDS address of a pointer into the workgroup's LDS
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Transposing LDS read (gfx950 ds_read_b64_tr_b16).  Within each group of 16 lanes, lane i receives
// word i % 4 of the 8 bytes addressed by lane 4 j + i / 4, for j = 0..3.  Issued as inline assembly
// because the compiler treats the builtin's read as depending on every direct-to-LDS copy still in
// flight and waits for all of them (vmcnt(0)) before it; here the copies a read depends on have
// been waited for explicitly before the stage barrier.  The result is valid only after
// wait_lds_all.
__device__ __forceinline__ u32x2_t ds_read_tr16_b64(uint32_t addr) {
  u32x2_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// Waits for every outstanding LDS read of the wavefront; the N fragments are tied to the wait, so no
// use of them is scheduled before it.
template <int N>
__device__ __forceinline__ void wait_lds_all(u32x2_t (&v)[N]) {
  static_assert(N == 2 || N == 4 || N == 8, "fragment count");
  if constexpr (N == 2) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]));
  } else if constexpr (N == 4) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
  } else {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]));
  }
}

__device__ __forceinline__ float wave_max_q(float v) {  // over the 4 lanes l, l^16, l^32, l^48
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float wave_sum_q(float v) {
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// bf16 <-> fp32 on 32-bit words (element order: low half first)
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ f32x4_t bf16x4_to_f32(u32x2_t w) {
  return f32x4_t{bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y)};
}
// two fp32 -> two bf16 (round to nearest even), `a` in the low half
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)a) | ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)b) << 16);
}

// Geometry of the prefix kernel for head size D.
template <int D>
struct Geo {
  static constexpr int kRowBytes = 2 * D;                         // one cache row (bf16)
  static constexpr int kChunks = D / 8;                           // 16-byte pieces per row
  static constexpr int kStageBytes = kKeyBlock * kRowBytes;       // one tensor, one stage
  static constexpr int kCopies = kStageBytes / (kWaves * 1024);   // 1 KiB copies per wavefront per tensor
  static constexpr int kRowsPerCopy = 1024 / kRowBytes;
  static constexpr int kRing = 4;                                 // stages resident in LDS
  static constexpr int kLds = kRing * 2 * kStageBytes;  // dynamic LDS (the block-table window is static)
  static constexpr int kDTiles = D / 32;                          // 16-wide d tiles per wavefront (half of D)
  static constexpr int kDChunks = D / 32;                         // 32-d MFMA steps of a score
  static_assert(kCopies >= 1 && kStageBytes % (kWaves * 1024) == 0, "stage must split into wave copies");
  static_assert(kDTiles >= 1, "head size too small");
  static_assert(kLds + kTablePages * 4 <= kMaxDynLds + 8 * 1024 - 256, "LDS budget");
  static_assert(2 * 4 * kDTiles * 64 * 16 + 2 * 4 * 64 * 8 <= kLds, "key-tile merge fits the ring");
  // The 16-byte piece of row n that lands at LDS position p is piece p ^ swz(n): 16 consecutive rows
  // read at one piece index then hit 16 distinct bank groups.
  __device__ static __forceinline__ int swz(int n) { return kChunks >= 16 ? (n & 15) : ((n >> 1) & 7); }
};

// One wavefront per SIMD (128 KiB of LDS per workgroup at D = 256): the whole register file is usable.
template <int D, int RT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void spec_prefix_kernel(
    AttnArgs a) {
  using Gm = Geo<D>;
  constexpr int kRing = Gm::kRing;
  constexpr int NJ = Gm::kCopies;
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ int32_t tbl[kTablePages];  // block-table entries of the current window

  const int split = blockIdx.x;
  const int b = blockIdx.y / a.HKV;
  const int hkv = blockIdx.y - b * a.HKV;
  const int seq = a.seq_lens[b];
  const int prefix = seq - a.Q > 0 ? seq - a.Q : 0;
  const int chunk = split_chunk(prefix, a.splits, a.min_chunk);
  const int n_active = prefix > 0 ? (prefix + chunk - 1) / chunk : 0;
  // Split s takes positions [s * chunk, min((s + 1) * chunk, prefix)); the last active split (split 0
  // when the prefix is empty) also takes this step's in-flight positions [prefix, seq).  Query qi sees
  // the positions up to seq - q_len + qi, which include the whole prefix, so one causal bound per
  // row covers both kinds of position.
  const int last_split = n_active > 0 ? n_active - 1 : 0;
  const int start = split * chunk;
  const int end = split == last_split ? seq : min(start + chunk, prefix);
  if (split > last_split || start >= end) {
    // no position here: the split's rows get log-sum-exp -inf, so the combine kernel can read every
    // split without knowing the sequence length (uniform: the whole workgroup leaves)
    const int64_t part = ((int64_t)blockIdx.y * a.splits + split) * a.R;
    for (int r = threadIdx.x; r < a.R; r += kThreads) a.lse_part[part + r] = -__builtin_inff();
    return;
  }

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int l16 = lane & 15;
  const int qg = lane >> 4;
  const int kh = wave & 1;   // key tile of each stage
  const int dh = wave >> 1;  // half of the head dimension

  // ---- packed query rows: B fragments of the score product (rows >= R repeat row R - 1) ----
  bf16x8_t qf[RT][Gm::kDChunks];
  int last[RT];  // last visible position of the lane's score row in each row tile
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = min(rt * 16 + l16, a.R - 1);
    const int qi = r / a.G;
    const int h = hkv * a.G + (r - qi * a.G);
    last[rt] = seq - a.Q + qi;
    const uint16_t* qrow = a.q + (int64_t)(b * a.Q + qi) * a.sq_t + (int64_t)h * a.sq_h + qg * 8;
#pragma unroll
    for (int c = 0; c < Gm::kDChunks; ++c) qf[rt][c] = *reinterpret_cast<const bf16x8_t*>(qrow + c * 32);
  }

  // ---- copy schedule: per stage, wavefront `wave` moves NJ KiB of K and NJ KiB of V.  Lane offsets
  // within a stage are fixed; per stage only the page bases change (computed in scalar registers) ----
  const int32_t* bt_row = a.bt + (int64_t)b * a.sbt;
  const char* kbytes = reinterpret_cast<const char*>(a.kc + (int64_t)hkv * a.sk_h);
  const char* vbytes = reinterpret_cast<const char*>(a.vc + (int64_t)hkv * a.sv_h);
  int row_of[NJ];
  uint32_t koff[NJ], voff[NJ], poff[NJ];  // byte offsets: row t's piece, and the piece in row 0
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int t = (wave * NJ + j) * Gm::kRowsPerCopy + lane / Gm::kChunks;
    const int piece = (lane % Gm::kChunks) ^ Gm::swz(t);
    row_of[j] = t;
    poff[j] = piece * 16;
    koff[j] = (uint32_t)(t * a.sk_t * 2) + poff[j];
    voff[j] = (uint32_t)(t * a.sv_t * 2) + poff[j];
  }

  // byte offsets (within a stage's V rows) of this lane's transposing reads, one per d tile
  uint32_t vt_off[Gm::kDTiles];
  {
    const int n = kh * 16 + 4 * (lane >> 4) + ((lane >> 2) & 3);
    const int q4 = lane & 3;
#pragma unroll
    for (int dt = 0; dt < Gm::kDTiles; ++dt) {
      const int d = (dh * Gm::kDTiles + dt) * 16 + 4 * q4;
      vt_off[dt] = (uint32_t)(n * Gm::kRowBytes + (((d >> 3) ^ Gm::swz(n)) << 4) + (d & 7) * 2);
    }
  }

  // online softmax state: m_ref is the row's exponent reference, moved only when a score exceeds it
  // by more than kRescale (log2 units), so the probabilities stay below 2^kRescale and the
  // accumulators are rarely rescaled; the result equals the running-maximum form up to rounding
  constexpr float kRescale = 8.f;
  float m_ref[RT], l_run[RT];
  f32x4_t o_acc[RT][Gm::kDTiles];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_ref[rt] = -__builtin_inff();
    l_run[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < Gm::kDTiles; ++dt) o_acc[rt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // The split is walked in windows of at most kTablePages pages (one window unless the split spans
  // more pages than that); each window's block-table entries are read into LDS first, so inside the
  // pipelined loop the only vector-memory instructions are the stage copies and the explicit vmcnt
  // waits below count exactly those.
  for (int wstart = start; wstart < end;) {
    const int p0 = wstart / a.page;
    const int wend = min(end, (p0 + kTablePages) * a.page);
    const int npg = (wend - 1) / a.page - p0 + 1;
    for (int i = threadIdx.x; i < npg; i += kThreads) tbl[i] = bt_row[p0 + i];
    wait_vmcnt<0>();  // the query loads too: nothing may be left in flight before the exact waits below
    __syncthreads();
    const int nst = (wend - wstart + kKeyBlock - 1) / kKeyBlock;

    // Stages are copied in order; the next one starts in page pg_n at in-page offset og_n.  A stage
    // of 32 positions spans at most 3 pages of >= 16 positions.
    int issued = 0, pg_n = p0, og_n = wstart - p0 * a.page;
    auto copy_next = [&]() {
      const int st = issued++;
      uint8_t* slot = lds + (st % kRing) * 2 * Gm::kStageBytes;
      const int nvalid = min(kKeyBlock, wend - (wstart + st * kKeyBlock));
      const int bnd1 = a.page - og_n;  // rows >= bnd1 lie in the next page, rows >= bnd2 in the one after
      const int bnd2 = bnd1 + a.page;
      const int e0 = pg_n - p0;
      const int64_t blk0 = __builtin_amdgcn_readfirstlane(tbl[e0]);
      const int64_t kb0 = (blk0 * a.sk_b + (int64_t)og_n * a.sk_t) * 2;
      const int64_t vb0 = (blk0 * a.sv_b + (int64_t)og_n * a.sv_t) * 2;
      if (bnd1 >= kKeyBlock && nvalid == kKeyBlock) {
        // the whole stage lies in one page (uniform): one base per tensor
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int copy = wave * NJ + j;
          __builtin_amdgcn_global_load_lds((gptr_t)(kbytes + kb0 + koff[j]), (lptr_t)(slot + copy * 1024), 16, 0, 0);
          __builtin_amdgcn_global_load_lds((gptr_t)(vbytes + vb0 + voff[j]),
                                           (lptr_t)(slot + Gm::kStageBytes + copy * 1024), 16, 0, 0);
        }
      } else {
        const int64_t blk1 = __builtin_amdgcn_readfirstlane(tbl[min(e0 + 1, npg - 1)]);
        const int64_t blk2 = __builtin_amdgcn_readfirstlane(tbl[min(e0 + 2, npg - 1)]);
        const int64_t kb1 = (blk1 * a.sk_b + (int64_t)(og_n - a.page) * a.sk_t) * 2;
        const int64_t kb2 = (blk2 * a.sk_b + (int64_t)(og_n - 2 * a.page) * a.sk_t) * 2;
        const int64_t vb1 = (blk1 * a.sv_b + (int64_t)(og_n - a.page) * a.sv_t) * 2;
        const int64_t vb2 = (blk2 * a.sv_b + (int64_t)(og_n - 2 * a.page) * a.sv_t) * 2;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const bool valid = row_of[j] < nvalid;  // rows past the window re-read the stage's first row
          const int t = valid ? row_of[j] : 0;
          const int64_t kb = t >= bnd2 ? kb2 : (t >= bnd1 ? kb1 : kb0);
          const int64_t vb = t >= bnd2 ? vb2 : (t >= bnd1 ? vb1 : vb0);
          const int copy = wave * NJ + j;
          __builtin_amdgcn_global_load_lds((gptr_t)(kbytes + kb + (valid ? koff[j] : poff[j])),
                                           (lptr_t)(slot + copy * 1024), 16, 0, 0);
          __builtin_amdgcn_global_load_lds((gptr_t)(vbytes + vb + (valid ? voff[j] : poff[j])),
                                           (lptr_t)(slot + Gm::kStageBytes + copy * 1024), 16, 0, 0);
        }
      }
      og_n += kKeyBlock;
      while (og_n >= a.page) {
        og_n -= a.page;
        ++pg_n;
      }
    };

    // prologue: stages 0 .. kRing-2 in flight
#pragma unroll
    for (int s = 0; s < kRing - 1; ++s)
      if (s < nst) copy_next();

    constexpr int kCopiesPerStage = 2 * NJ;  // vector-memory instructions of one stage
    for (int st = 0; st < nst; ++st) {
      // Stage st has landed once at most the later issued stages' copies are outstanding.  Stages
      // up to st + kRing - 2 have been issued; st + kRing - 1 goes out after the barrier below.
      const int after = min(kRing - 2, nst - 1 - st);
      if (after >= 2) {
        wait_vmcnt<2 * kCopiesPerStage>();
      } else if (after == 1) {
        wait_vmcnt<kCopiesPerStage>();
      } else {
        wait_vmcnt<0>();
      }
      ring_barrier();
      // Refill the slot every wavefront finished with before this barrier (stage st - 1's); three
      // stages are then in flight while this one is computed.
      if (st + kRing - 1 < nst) copy_next();
      __builtin_amdgcn_sched_barrier(0);

      const uint8_t* ks = lds + (st % kRing) * 2 * Gm::kStageBytes;
      const uint8_t* vs = ks + Gm::kStageBytes;
      const int sbase = wstart + st * kKeyBlock;

      // S^T tile of this wavefront's key tile kh: positions 16 kh + 4 qg + i, row 16 rt + l16
      f32x4_t sc[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) sc[rt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const int n_k = kh * 16 + l16;
#pragma unroll
      for (int c = 0; c < Gm::kDChunks; ++c) {
        const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(
            ks + n_k * Gm::kRowBytes + (((4 * c + qg) ^ Gm::swz(n_k)) << 4));
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          sc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[rt][c], sc[rt], 0, 0, 0);
      }

      // softmax weights in base 2; the lane's 4 probabilities are its B fragment of O^T = V^T P^T.
      // A stage wholly inside every row's visible range needs no mask.
      const int pos0 = sbase + kh * 16 + qg * 4;
      const bool full = sbase + kKeyBlock <= wend && sbase + kKeyBlock - 1 <= seq - a.Q;
      s16x4_t pf[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        float v[4];
        if (full) {
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = sc[rt][i] * a.qk_scale;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            v[i] = pos0 + i < wend && pos0 + i <= last[rt] ? sc[rt][i] * a.qk_scale : -__builtin_inff();
        }
        const float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
        if (__any(mx > m_ref[rt] + kRescale)) {  // wave-uniform: move the references of all rows
          const float m_new = fmaxf(m_ref[rt], wave_max_q(mx));
          // -inf only for a row that has seen no position yet: exponent base 0 then
          const float alpha = fast_exp2(m_ref[rt] - (m_new == -__builtin_inff() ? 0.f : m_new));
          l_run[rt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < Gm::kDTiles; ++dt) o_acc[rt][dt] *= alpha;
          m_ref[rt] = m_new;
        }
        const float m_base = m_ref[rt] == -__builtin_inff() ? 0.f : m_ref[rt];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = fast_exp2(v[i] - m_base);
        l_run[rt] += (v[0] + v[1]) + (v[2] + v[3]);
        pf[rt] = __builtin_bit_cast(s16x4_t, u32x2_t{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])});
      }

      // O^T += V^T P^T over this wavefront's d half and key tile (k slot 4 qg + i = position 4 qg + i).
      // The V^T fragment of a d tile comes from one transposing LDS read: lane 16 g + 4 j + q points at
      // the 8 bytes of row 4 g + j holding d values d0 + 4 q .. d0 + 4 q + 3, and the read hands lane
      // 16 g + i the values V[4 g + j][d0 + i], j = 0..3.
      u32x2_t vf[Gm::kDTiles];
      const uint32_t vs_lds = lds_addr(vs);
#pragma unroll
      for (int dt = 0; dt < Gm::kDTiles; ++dt) vf[dt] = ds_read_tr16_b64(vs_lds + vt_off[dt]);
      wait_lds_all<Gm::kDTiles>(vf);
#pragma unroll
      for (int dt = 0; dt < Gm::kDTiles; ++dt) {
        const s16x4_t a_frag = __builtin_bit_cast(s16x4_t, vf[dt]);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          o_acc[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a_frag, pf[rt], o_acc[rt][dt], 0, 0, 0);
      }
    }
    wait_vmcnt<0>();
    __syncthreads();  // the next window rewrites the table and the ring
    wstart = wend;
  }

  // ---- merge the two key tiles' states (wavefront kh = 1 hands its state to kh = 0 of the same d
  // half through the now idle ring), then the partial output (normalised) and base-2 log-sum-exp of
  // each packed row; a row that saw no position (possible only in the split holding the in-flight
  // positions) is written as 0 with log-sum-exp -inf ----
  float* xo = reinterpret_cast<float*>(lds);                        // [2][RT][kDTiles][64] x f32x4
  float* xs = xo + 2 * RT * Gm::kDTiles * kWave * 4;               // [2][RT][64] x (m, l)
  float l_tot[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) l_tot[rt] = wave_sum_q(l_run[rt]);
  if (kh == 1) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int dt = 0; dt < Gm::kDTiles; ++dt)
        *reinterpret_cast<f32x4_t*>(xo + (((dh * RT + rt) * Gm::kDTiles + dt) * kWave + lane) * 4) = o_acc[rt][dt];
      xs[((dh * RT + rt) * kWave + lane) * 2] = m_ref[rt];
      xs[((dh * RT + rt) * kWave + lane) * 2 + 1] = l_tot[rt];
    }
  }
  __syncthreads();
  if (kh == 1) return;
  const int64_t part = ((int64_t)blockIdx.y * a.splits + split) * a.R;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float m1 = xs[((dh * RT + rt) * kWave + lane) * 2];
    const float l1 = xs[((dh * RT + rt) * kWave + lane) * 2 + 1];
    const float mt = fmaxf(m_ref[rt], m1);
    const float mb = mt == -__builtin_inff() ? 0.f : mt;
    const float a0 = fast_exp2(m_ref[rt] - mb), a1 = fast_exp2(m1 - mb);
    const float lt = l_tot[rt] * a0 + l1 * a1;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int r = rt * 16 + l16;
    if (r < a.R) {
      float* orow = a.o_part + (part + r) * D;
#pragma unroll
      for (int dt = 0; dt < Gm::kDTiles; ++dt) {
        const f32x4_t o1 =
            *reinterpret_cast<const f32x4_t*>(xo + (((dh * RT + rt) * Gm::kDTiles + dt) * kWave + lane) * 4);
        *reinterpret_cast<f32x4_t*>(orow + (dh * Gm::kDTiles + dt) * 16 + qg * 4) =
            (o_acc[rt][dt] * a0 + o1 * a1) * inv;
      }
      if (dh == 0 && qg == 0) a.lse_part[part + r] = lt > 0.f ? mt + __log2f(lt) : -__builtin_inff();
    }
  }
}

// One workgroup per (token, head, 64-wide slice of d): the row's split partials merged by log-sum-exp
// (the merge of the reference's _suffix_combine_kernel, spec_attn.py:119-131).  Every split has
// written its rows' log-sum-exp (-inf where it saw nothing), so all loads issue at once, with no
// dependence on the sequence length; 16 groups of 16 threads merge every 16th split, then LDS merges
// the groups.
constexpr int kCombSlice = 64;  // d values per combine workgroup

template <int D>
__global__ __launch_bounds__(kThreads) void spec_combine_kernel(AttnArgs a) {
  constexpr int NQ = kCombSlice / 4;  // threads per group, 4 d values each
  constexpr int NGRP = kThreads / NQ;
  constexpr int kBatch = 4;           // parts a thread loads before merging them
  __shared__ float sm_m[NGRP], sm_l[NGRP];
  __shared__ __align__(16) float sm_acc[NGRP][kCombSlice];

  const int row = blockIdx.x;
  const int d0 = blockIdx.y * kCombSlice;
  const int tok = row / a.H;
  const int h = row - tok * a.H;
  const int b = tok / a.Q;
  const int qi = tok - b * a.Q;
  const int hkv = h / a.G;
  const int r = qi * a.G + (h - hkv * a.G);
  const int grp = threadIdx.x / NQ;
  const int dq = threadIdx.x - grp * NQ;

  float m = -__builtin_inff(), l = 0.f;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  const int64_t part0 = ((int64_t)(b * a.HKV + hkv) * a.splits) * a.R + r;
  // group grp merges the parts grp, grp + NGRP, ...
  for (int base = grp; base < a.splits; base += NGRP * kBatch) {
    float e[kBatch];
    f32x4_t o[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int i = base + u * NGRP;
      e[u] = -__builtin_inff();
      if (i < a.splits) {
        const int64_t idx = part0 + (int64_t)i * a.R;
        e[u] = a.lse_part[idx];
        o[u] = *reinterpret_cast<const f32x4_t*>(a.o_part + idx * D + d0 + dq * 4);
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (e[u] == -__builtin_inff()) continue;  // a split with no position, or a row that saw none
      const float mn = fmaxf(m, e[u]);
      const float c_old = fast_exp2(m - mn);
      const float w = fast_exp2(e[u] - mn);
      acc = acc * c_old + o[u] * w;
      l = l * c_old + w;
      m = mn;
    }
  }

  if (dq == 0) {
    sm_m[grp] = m;
    sm_l[grp] = l;
  }
  *reinterpret_cast<f32x4_t*>(&sm_acc[grp][dq * 4]) = acc;
  __syncthreads();
  if (grp != 0) return;
  float mt = -__builtin_inff();
#pragma unroll
  for (int g = 0; g < NGRP; ++g) mt = fmaxf(mt, sm_m[g]);
  f32x4_t at = {0.f, 0.f, 0.f, 0.f};
  float lt = 0.f;
  if (mt != -__builtin_inff()) {
#pragma unroll
    for (int g = 0; g < NGRP; ++g) {
      const float w = fast_exp2(sm_m[g] - mt);  // 0 for an empty group
      at += *reinterpret_cast<const f32x4_t*>(&sm_acc[g][dq * 4]) * w;
      lt += sm_l[g] * w;
    }
  }
  const float inv = lt > 0.f ? 1.f / lt : 0.f;  // a row that sees no position is written as zeros
  *reinterpret_cast<u32x2_t*>(a.out + (int64_t)tok * a.so_t + (int64_t)h * a.so_h + d0 + dq * 4) =
      u32x2_t{pack_bf16(at[0] * inv, at[1] * inv), pack_bf16(at[2] * inv, at[3] * inv)};
}

typedef void (*KernelFn)(AttnArgs);

template <int D>
KernelFn prefix_fn(int rt) {
  switch (rt) {
    case 1: return &spec_prefix_kernel<D, 1>;
    case 2: return &spec_prefix_kernel<D, 2>;
    case 3: return &spec_prefix_kernel<D, 3>;
    case 4: return &spec_prefix_kernel<D, 4>;
    default: return nullptr;
  }
}

std::mutex g_lds_mutex;
std::unordered_set<const void*> g_lds_raised;

int launch(KernelFn fn, dim3 grid, size_t smem, hipStream_t stream, const AttnArgs& a) {
  void* args[] = {const_cast<AttnArgs*>(&a)};
  if (smem > kDefaultLds) {
    std::lock_guard<std::mutex> lock(g_lds_mutex);
    const void* key = reinterpret_cast<const void*>(fn);
    if (g_lds_raised.find(key) == g_lds_raised.end()) {
      if (hipFuncSetAttribute(key, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxDynLds) != hipSuccess)
        return QF_ERR_HIP;
      g_lds_raised.insert(key);
    }
  }
  if (hipLaunchKernel(reinterpret_cast<const void*>(fn), grid, dim3(kThreads), args, smem, stream) != hipSuccess)
    return QF_ERR_HIP;
  return QF_OK;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

size_t workspace_for(int B, int Q, int H, int HKV, int D, int S) {
  if (B < 1 || Q < 1 || H < 1 || HKV < 1 || H % HKV || D < 1 || S < 1) return 0;
  const size_t R = (size_t)Q * (H / HKV);
  const size_t n = (size_t)B * HKV * S * R * (D + 1) * sizeof(float);
  return (n + 255) / 256 * 256;
}

}  // namespace qfa

using namespace qfa;

extern "C" {

int qf_spec_attn_abi_version(void) { return QF_SPEC_ATTN_ABI_VERSION; }

size_t qf_spec_attn_workspace_bytes(int num_reqs, int q_len, int num_heads, int num_kv_heads, int head_size,
                                    int num_splits) {
  return workspace_for(num_reqs, q_len, num_heads, num_kv_heads, head_size, num_splits);
}

int qf_spec_attention(const uint16_t* query, int64_t q_stride_tok, int64_t q_stride_head,
                      const uint16_t* key_cache, int64_t k_stride_block, int64_t k_stride_tok,
                      int64_t k_stride_head,
                      const uint16_t* value_cache, int64_t v_stride_block, int64_t v_stride_tok,
                      int64_t v_stride_head,
                      const int32_t* block_table, int64_t bt_stride,
                      const int32_t* seq_lens,
                      uint16_t* out, int64_t o_stride_tok, int64_t o_stride_head,
                      int num_reqs, int q_len, int num_heads, int num_kv_heads, int head_size,
                      int page_size, float scale, int num_splits, int min_chunk,
                      void* workspace, size_t workspace_bytes, void* stream) {
  if (!query || !key_cache || !value_cache || !block_table || !seq_lens || !out) return QF_ERR_INVALID_ARG;
  if (num_reqs < 1 || q_len < 1 || num_heads < 1 || num_kv_heads < 1 || page_size < 1 || num_splits < 1 ||
      num_splits > 65535 || min_chunk < 1 || bt_stride < 0)
    return QF_ERR_INVALID_ARG;
  if (!(scale == scale)) return QF_ERR_INVALID_ARG;
  if (num_heads % num_kv_heads) return QF_ERR_UNSUPPORTED;
  const int G = num_heads / num_kv_heads;
  const int R = q_len * G;
  if (R > kMaxRows || page_size < QF_SPEC_ATTN_MIN_PAGE) return QF_ERR_UNSUPPORTED;
  if (head_size != 64 && head_size != 128 && head_size != 256) return QF_ERR_UNSUPPORTED;
  if ((int64_t)num_reqs * num_kv_heads > 65535 || (int64_t)num_reqs * q_len * num_heads > 0x7fffffff)
    return QF_ERR_UNSUPPORTED;
  const int64_t strides[] = {q_stride_tok, q_stride_head, k_stride_block, k_stride_tok, k_stride_head,
                             v_stride_block, v_stride_tok, v_stride_head, o_stride_tok, o_stride_head};
  for (int64_t s : strides)
    if (s < 0 || s % 8) return QF_ERR_UNSUPPORTED;
  // the prefix kernel keeps per-lane byte offsets of up to one stage of rows in 32 bits
  if ((k_stride_tok > v_stride_tok ? k_stride_tok : v_stride_tok) * 2 * kKeyBlock >= ((int64_t)1 << 31))
    return QF_ERR_UNSUPPORTED;
  if (!aligned16(query) || !aligned16(key_cache) || !aligned16(value_cache) || !aligned16(out))
    return QF_ERR_UNSUPPORTED;
  const size_t need = workspace_for(num_reqs, q_len, num_heads, num_kv_heads, head_size, num_splits);
  if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)) return QF_ERR_WORKSPACE;

  AttnArgs a;
  a.q = query;
  a.sq_t = q_stride_tok;
  a.sq_h = q_stride_head;
  a.kc = key_cache;
  a.sk_b = k_stride_block;
  a.sk_t = k_stride_tok;
  a.sk_h = k_stride_head;
  a.vc = value_cache;
  a.sv_b = v_stride_block;
  a.sv_t = v_stride_tok;
  a.sv_h = v_stride_head;
  a.bt = block_table;
  a.sbt = bt_stride;
  a.seq_lens = seq_lens;
  a.out = out;
  a.so_t = o_stride_tok;
  a.so_h = o_stride_head;
  const size_t n_o = (size_t)num_reqs * num_kv_heads * num_splits * R * head_size;
  a.o_part = static_cast<float*>(workspace);
  a.lse_part = a.o_part + n_o;
  a.B = num_reqs;
  a.Q = q_len;
  a.H = num_heads;
  a.HKV = num_kv_heads;
  a.G = G;
  a.R = R;
  a.page = page_size;
  a.splits = num_splits;
  a.min_chunk = min_chunk;
  a.qk_scale = scale * kLog2e;

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rt = (R + 15) / 16;
  KernelFn pre = nullptr, comb = nullptr;
  size_t lds = 0;
  switch (head_size) {
    case 64: pre = prefix_fn<64>(rt); comb = &spec_combine_kernel<64>; lds = Geo<64>::kLds; break;
    case 128: pre = prefix_fn<128>(rt); comb = &spec_combine_kernel<128>; lds = Geo<128>::kLds; break;
    default: pre = prefix_fn<256>(rt); comb = &spec_combine_kernel<256>; lds = Geo<256>::kLds; break;
  }
  if (pre == nullptr) return QF_ERR_UNSUPPORTED;
  int st = launch(pre, dim3(num_splits, num_reqs * num_kv_heads), lds, s, a);
  if (st != QF_OK) return st;
  return launch(comb, dim3(num_reqs * q_len * num_heads, head_size / kCombSlice), 0, s, a);
}

}  // extern "C"
