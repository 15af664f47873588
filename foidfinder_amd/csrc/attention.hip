// Non-causal flash attention, head_dim 64, fp16 in / fp32 accumulate, on gfx950 fp16 MFMA.
//
// Input is the QKV GEMM's output: qkv fp16 [S*L, 3C] with q already rotated and scaled by softmax_scale*log2(e) and
// k rotated, so the softmax is in base 2. One 256-thread workgroup = 4 waves x 32 queries (one 32-query tile per
// wave) of one (sequence, head); four workgroups share a CU (16 waves, 4 per SIMD), so one wave's softmax (VALU)
// runs beside the other waves' MFMA products.
//
// K and V stream through a 2-stage LDS ring of 64-key tiles filled by buffer loads straight into LDS
// (buffer_load_dwordx4 ... lds: no VGPR staging, no LDS write instructions). The buffer descriptor of each tile ends
// at the sequence's last row, so rows past L read as zeros without any address clamping. Both tiles are stored
// row-major (64 keys x 128 B); K is read with ds_read_b128 and V with the transposing ds_read_b64_tr_b16, which
// hands each lane 4 consecutive keys of one d column - the layout the PV MFMA wants - so V is never transposed in
// software. Rows are XOR-swizzled in 16-byte chunks so that both read patterns are free of bank conflicts.
//
// Per wave, S^T = K Q^T comes from v_mfma_f32_32x32x16_f16 with each lane holding one query and 16 of every 32 keys
// (the other 16 sit in lane ^ 32), and P^T feeds the PV MFMA (O^T = V^T P^T) directly as its column operand. The
// tile is processed in two 32-key halves (S, softmax, PV per half). At head_dim 64 the softmax, not the MFMA, bounds
// the loop, so its common path is one exp2, half a convert and half a packed add per score:
//  * every S^T accumulator starts at -m_ref (the query's reference maximum, kept fp16-representable): a register
//    block holding -m_ref is the C operand of each half's first product; the first tile's first key half sets m_ref
//    to its maximum;
//  * p = v_exp_f32 (exp2), converted in pairs to fp16 for the PV product; each lane sums those fp16 p (the weights the
//    PV product applies) by a pairwise tree of v_pk_add_f16 (7 packed adds per 16 p) and one exact fp32 add of the
//    last pair, and the half sums accumulate in fp32. The tree rounds to fp16 at each level (relative error at most
//    ~4 x 2^-11 per half sum, unbiased); it replaced 16 fp32 adds per half (1.3 % faster at 32 x 16 x 1025). A v_dot2
//    on the fp16 pairs would share the matrix core's issue and stall behind its products. While every lane's sum over
//    a half stays <= SUM_LIMIT, every p <= SUM_LIMIT, which fp16 holds at full relative precision, so m_ref stays (a
//    sum past fp16's range reads as infinity and takes the rescue path). Otherwise (rare: the scores rose well above
//    m_ref) m_ref is raised to that half's
//    maximum, O and l are rescaled by 2^(m_old - m_new) and the half's p are recomputed.
// Tails: query rows >= L are computed on clamped rows and not stored; keys >= L (zero K rows) get S ~ -2^17 from
// an extra MFMA in the last tile (see last_operands below), so their p is exactly 0 with no masking instructions; when
// the last tile's second half holds no key below L it is skipped. The last query block of a sequence, when it holds
// two 32-query units, gives each unit two waves, one per key half; when it holds one (L = 1025 leaves one query), all
// four waves share it, each over one key half of every other tile. The partial results are merged through LDS at the
// end, so that block takes about a quarter of a block's time instead of a whole block's with three waves idle. A grid
// of 128-query blocks that fills at most half of the GPU's resident workgroups (batch 1 and 2) runs as 64-query blocks
// instead, each unit over two waves by key half: twice the workgroups.
//
// Reference: foidfinder/backends/cuda/csrc/attention.cuh:19-157 (which accumulates each 64-key block in fp16 and
// rescales every block; here every product and sum is fp32).
#include <type_traits>

#include "common.h"

namespace ff {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int HD = 64;
constexpr int QW = 32;                // queries per wave
constexpr int WAVES = 4;              // waves per workgroup
constexpr int BQ = WAVES * QW;        // queries per workgroup
constexpr int BKV = 64;               // keys per tile
constexpr int STAGES = 2;             // LDS ring depth
constexpr int TILE = BKV * HD;        // halves per K (or V) tile: 8 KB
constexpr int KPW = 8 / WAVES;        // 1 KB blocks of each K (and V) tile loaded per wave
constexpr int LOADS = 2 * KPW;        // buffer->LDS loads per thread per tile
constexpr float SUM_LIMIT = 8192.f;   // per-lane half-tile sum of p above which m_ref is raised
constexpr uint32_t RSRC_WORD3 = 0x00020000;  // buffer descriptor word 3: raw dword access (gfx9 family)
constexpr int MERGE_WORDS = 34;       // floats per lane of a merged wave's partial result: O (32), m_ref, l
static_assert((WAVES - 1) * MERGE_WORDS * 64 * 4 <= 2 * STAGES * TILE * 2, "merge area exceeds the LDS ring");

// Physical 16-byte slot of chunk c in row r. K rows are read 16 rows per ds_read_b128 pass: XOR with bits 1-3 of the
// row spreads them over all 64 banks. V rows are read by the transposing b64 read, 4 rows x 64 B per 32-lane pass:
// flipping the upper half of the row for rows 2, 3 (mod 4) keeps those 4 rows on distinct banks.
__device__ __forceinline__ int k_slot(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ int v_slot(int r, int c) { return c ^ ((r & 2) << 1); }

// ds_read_b64_tr_b16 as inline asm. The compiler's wait-insertion pass treats the builtin as possibly reading LDS
// that in-flight buffer->LDS loads are writing and drains them all (s_waitcnt vmcnt(0)) before it, which would
// serialize the LDS ring; this form is invisible to that pass. Ordering: "memory" keeps it after the barrier that
// publishes the tile; the caller waits for the data (s_waitcnt lgkmcnt(0) tied to the result registers).
template <int OFF>
__device__ __forceinline__ void tr_read(half4_t& v, uint32_t lds_addr) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(lds_addr), "n"(OFF) : "memory");
}

// One workgroup's work, the queries from q_first. SPLIT = 0: wave w owns queries q_first + 32w .. +31 over both
// key halves of every tile.
// SPLIT = 1 (last block of two units): waves 2u and 2u + 1 share query unit u, each over one key half (kh_sel = w & 1);
// the half-1 wave's O, m_ref and l are merged into its partner's at the end. SPLIT = 2 (last block of one unit): all
// four waves share unit 0, wave w over key half w & 1 of the tiles of parity w >> 1; waves 1-3 are merged into wave 0.
template <int SPLIT>
__device__ __forceinline__ void attention_block(const half_t* __restrict__ qkv, half_t* __restrict__ out, int L,
                                                int H, int q_first, int h, int seq, half_t* smem) {
  const uint32_t smem_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)smem));
  const int C = H * HD, ROW = 3 * C;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fh = lane >> 5;
  const int64_t tok0 = static_cast<int64_t>(seq) * L;
  const half_t* qbase = qkv + tok0 * ROW + h * HD;
  const half_t* kbase = qbase + C;
  const half_t* vbase = qbase + 2 * C;

  const int unit = SPLIT == 2 ? 0 : (SPLIT ? wave >> 1 : wave);
  const int kh_sel = SPLIT ? wave & 1 : 0;
  const int first_tile = SPLIT == 2 ? wave >> 1 : 0;  // SPLIT 2: the wave computes tiles first_tile, +2, ...
  bool seen = false;                                   // the wave has computed a tile (it has keys to merge)
  const int q0 = q_first + unit * QW;
  const bool active = q0 < L;  // a wave whose queries all lie past L only helps load K and V
  const int ntiles = (L + BKV - 1) / BKV;
  const bool h1_empty = (ntiles - 1) * BKV + 32 >= L;  // the last tile's keys 32..63 all lie past L

  // Q fragments (column operand of S^T): lane holds query q0 + fr, d = 16s + 8fh + 0..7.
  half8_t qf[4];
  {
    const int qrow = min(q0 + fr, L - 1);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qf[s] = *reinterpret_cast<const half8_t*>(qbase + static_cast<int64_t>(qrow) * ROW + 16 * s + 8 * fh);
  }
  // Consume Q here, so that the compiler's own wait for these loads is placed once, before the tile loop, and not
  // inside it, where the same vmcnt counter also tracks the tile loads in flight.
#pragma unroll
  for (int s = 0; s < 4; ++s) asm volatile("" ::"v"(qf[s]));

  // Tile loads: wave w fills the 1 KB blocks KPW*w .. KPW*w + KPW-1 of each tile (8 rows each); lane l writes LDS
  // slot l of the block, so it fetches the chunk that the swizzle puts there.
  uint32_t voff_k[KPW], voff_v[KPW];
#pragma unroll
  for (int p = 0; p < KPW; ++p) {
    const int row = 8 * (KPW * wave + p) + (lane >> 3), slot = lane & 7;
    voff_k[p] = static_cast<uint32_t>((row * ROW + k_slot(row, slot) * 8) * 2);
    voff_v[p] = static_cast<uint32_t>((row * ROW + v_slot(row, slot) * 8) * 2);
  }
  auto issue = [&](int tile) __attribute__((always_inline)) {
    const int st = tile % STAGES;
    const int64_t off = static_cast<int64_t>(tile) * BKV * ROW;
    const int nrec = ((L - 1 - tile * BKV) * ROW + HD) * 2;  // bytes up to the end of the sequence's last row
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(kbase + off), 0, nrec, RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(vbase + off), 0, nrec, RSRC_WORD3);
#pragma unroll
    for (int p = 0; p < KPW; ++p) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(smem + st * TILE + (KPW * wave + p) * 512), 16,
                                               voff_k[p], 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(smem + (STAGES + st) * TILE + (KPW * wave + p) * 512),
                                               16, voff_v[p], 0, 0, 0);
    }
  };

  // LDS read offsets (halves, within a tile). K fragment (kh, s): row kh*32 + fr, chunk 2s + fh. V^T fragment
  // (dt, kh, tt), half j: the transposing read over 16-lane groups; lane l of group g addresses row
  // kh*32 + 16tt + 8j + 4fh + (l%16)/4, columns dt*32 + 16(g%2) + 4(l%4) .. +3, and receives 4 consecutive keys of
  // column dt*32 + fr: MFMA slots 4j .. 4j+3 = keys 16tt + 8j + 4fh + 0..3, the keys of P^T's slots. A SPLIT wave's
  // rows start at its own half (kh_sel*32).
  int koff[4], voff[2];
#pragma unroll
  for (int s = 0; s < 4; ++s) koff[s] = fr * HD + k_slot(fr, 2 * s + fh) * 8 + kh_sel * 32 * HD;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    const int row = 4 * fh + ((lane & 15) >> 2);  // + kh*32 + 16tt + 8j, multiples of 4 that leave row & 2 alone
    const int col = dt * 32 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    voff[dt] = row * HD + v_slot(row, col >> 3) * 8 + (col & 7) + kh_sel * 32 * HD;
  }

  float16_t o[2];  // [d tile]: O^T rows d = 32dt + 8(r/4) + 4fh + r%4, column = the lane's query
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  float m_ref = 0.f, l_run = 0.f;
  half_t m_ref_h = static_cast<half_t>(0.f);
  float16_t negm = {};  // -m_ref in every accumulator slot (the lane's query)
  auto set_mref = [&](float m) __attribute__((always_inline)) {
    // smallest fp16 >= m (|m| < 65504): then every p of the tile that set it is <= 1
    const float mc = fminf(fmaxf(m, -65000.f), 65000.f);
    m_ref_h = static_cast<half_t>(mc + fabsf(mc) * 0.0009765625f + 6.103515625e-05f);
    m_ref = static_cast<float>(m_ref_h);
#pragma unroll
    for (int r = 0; r < 16; ++r) negm[r] = -m_ref;
  };
  // m_ref enters S as the C operand of each half's first product: negm holds -m_ref in every accumulator slot (the
  // lane's query), kept fp16-representable (|m_ref| <= 65000). The last tile instead starts each half with one extra
  // MFMA whose row operand has 1 in k-slot 0 for every key and 2 in k-slot 1 for keys >= L, against -m_ref and
  // -65504 in the column operand's k-slots 0 and 1: keys past the sequence start at -m_ref - 131008 < -66000, so
  // exp2 gives exactly 0 (their K rows are zero), with no per-score select. Those operands are built in the last
  // tile only (no registers held through the loop).
  auto last_operands = [&](int kh, half8_t& ok, half8_t& mq) __attribute__((always_inline)) {
    ok = {};
    mq = {};
    if (fh == 0) {
      ok[0] = static_cast<half_t>(1.f);
      // key of this lane's row in the last tile: half kh (SPLIT: slot 0 is the wave's own half kh_sel)
      const int key = (ntiles - 1) * BKV + (SPLIT ? kh_sel : kh) * 32 + fr;
      ok[1] = static_cast<half_t>(key >= L ? 2.f : 0.f);
      mq[0] = static_cast<half_t>(-m_ref_h);
      mq[1] = static_cast<half_t>(-65504.f);
    }
  };

  // One half's S and p at a time (the halves run one after the other, so one register block each suffices)
  float16_t xs;    // S^T - m_ref of the current half kh: lane holds keys 32kh + 8(r/4) + 4fh + r%4
  half8_t pf[2];   // [tt]: fp16 p, slot u of lane half fh = key 32kh + 16tt + 8(u/4) + 4fh + u%4
  float hs[2];     // [kh]: the lane's sum of its p over half kh
  int ka[4], va[2];  // this tile's K and V read bases

  // Half kh of the tile (SPLIT: slot 0 is the wave's own half, whose rows koff/voff already select)
  auto qk = [&](int kh, auto lastc) __attribute__((always_inline)) {
    if constexpr (decltype(lastc)::value) {
      const float16_t zero = {};
      half8_t ok, mq;
      last_operands(kh, ok, mq);
      xs = __builtin_amdgcn_mfma_f32_32x32x16_f16(ok, mq, zero, 0, 0, 0);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const half8_t kf = *reinterpret_cast<const half8_t*>(smem + ka[s] + kh * 32 * HD);
        xs = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], xs, 0, 0, 0);
      }
    } else {
      // every other tile: -m_ref enters as the C operand of the first product (no extra MFMA)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const half8_t kf = *reinterpret_cast<const half8_t*>(smem + ka[s] + kh * 32 * HD);
        xs = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], s == 0 ? negm : xs, 0, 0, 0);
      }
    }
  };
  auto soft = [&](int kh) __attribute__((always_inline)) {
    // p in fp16 pairs, summed by a pairwise tree of packed fp16 adds (7 per 16 p) and one fp32 add of the last pair
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const float e0 = __builtin_amdgcn_exp2f(xs[r]), e1 = __builtin_amdgcn_exp2f(xs[r + 1]);
      pf[r >> 3][r & 7] = static_cast<half_t>(e0);
      pf[r >> 3][(r & 7) + 1] = static_cast<half_t>(e1);
    }
    half2_t a[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) a[k] = half2_t{pf[k >> 2][2 * (k & 3)], pf[k >> 2][2 * (k & 3) + 1]};
#pragma unroll
    for (int w = 4; w >= 1; w >>= 1)
#pragma unroll
      for (int k = 0; k < w; ++k) a[k] = a[k] + a[k + w];
    // the last pair's two halves as one fp32 sum (exact: fp16 operands, one rounding)
    float sum;
    asm("v_fma_mix_f32 %0, %1, 1.0, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(sum) : "v"(a[0]));
    hs[kh] = sum;
  };
  auto pv = [&](auto khc) __attribute__((always_inline)) {
    constexpr int kh = decltype(khc)::value;
    half4_t v[2][2][2];  // [dt][tt][j]
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const uint32_t base = smem_lds + 2u * static_cast<uint32_t>(va[dt]);
      tr_read<(kh * 32 + 0) * HD * 2>(v[dt][0][0], base);
      tr_read<(kh * 32 + 8) * HD * 2>(v[dt][0][1], base);
      tr_read<(kh * 32 + 16) * HD * 2>(v[dt][1][0], base);
      tr_read<(kh * 32 + 24) * HD * 2>(v[dt][1][1], base);
    }
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0][0][0]), "+v"(v[0][0][1]), "+v"(v[0][1][0]), "+v"(v[0][1][1]), "+v"(v[1][0][0]),
                   "+v"(v[1][0][1]), "+v"(v[1][1][0]), "+v"(v[1][1][1]));
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const half4_t lo = v[dt][tt][0], hi = v[dt][tt][1];
        const half8_t vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[tt], o[dt], 0, 0, 0);
      }
  };
  // Lane-pair maximum of xs (the query's 32 keys of the current half).
  auto half_max = [&]() __attribute__((always_inline)) {
    float v = xs[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) v = fmaxf(v, xs[r]);
    return fmaxf(v, xor_shuffle(v, 32));
  };
  // Rare path of a half whose p overflowed the limit: raise m_ref to the maximum of S over that half (S recomputed
  // under the old m_ref), rescale O, l and the sum of half 0 when rescuing half 1, and recompute the half's S and p
  // under the new m_ref.
  auto rescue = [&](int kh, auto lastc) __attribute__((always_inline)) {
    qk(kh, lastc);
    const float m_old = m_ref;
    const float mx = half_max() + m_old;
    if (mx > m_old) set_mref(mx);
    const float corr = __builtin_amdgcn_exp2f(m_old - m_ref);
    l_run *= corr;
    if (kh == 1) hs[0] *= corr;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] *= corr;
    qk(kh, lastc);
    soft(kh);
  };

#pragma unroll
  for (int j = 0; j < STAGES - 1; ++j)
    if (j < ntiles) issue(j);
  // One tile. LAST (the final tile, whose keys past L are masked by the extra MFMA) is a separate copy of the code,
  // so the other tiles take -m_ref through the first product's C operand without a branch in their loop.
  auto tile_body = [&](int tile, auto lastc) __attribute__((always_inline)) {
    constexpr bool LAST = decltype(lastc)::value;
    // Tile `tile` has landed once at most the loads of the tiles issued after it are outstanding.
    if (tile + 1 < ntiles && STAGES > 2)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS * (STAGES - 2)) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();  // no fence: the vmcnt wait above already covers this thread's LDS writes
    // The ring slot of tile + STAGES - 1 was last read for tile - 1, which every wave has finished.
    if (tile + STAGES - 1 < ntiles) issue(tile + STAGES - 1);
    if (!active || (SPLIT && LAST && kh_sel == 1 && h1_empty)) return;
    if (SPLIT == 2 && (tile & 1) != first_tile) return;
    // Read bases, opaque to the compiler so that the fragment offsets fold into the reads' immediate offsets
    // instead of each being precomputed into a register.
    const int st = tile % STAGES;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      ka[s] = st * TILE + koff[s];
      asm volatile("" : "+v"(ka[s]));
    }
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      va[dt] = (STAGES + st) * TILE + voff[dt];
      asm volatile("" : "+v"(va[dt]));
    }
    // Each half's p are checked (all lane sums <= SUM_LIMIT) before its PV product. The wave's first tile sets m_ref
    // from the maximum of its first half (one extra S product per wave; the second half, like every later one, takes
    // the rescue path if its scores rise well above it). From both halves' maximum it cost a second extra product and
    // ran ~0.7 % slower.
    if (tile == first_tile) {
      qk(0, lastc);
      set_mref(half_max());
    }
    qk(0, lastc);
    soft(0);
    if (__any(hs[0] > SUM_LIMIT)) rescue(0, lastc);
    pv(std::integral_constant<int, 0>{});
    hs[1] = 0.f;
    if (!SPLIT && !(LAST && h1_empty)) {
      qk(1, lastc);
      soft(1);
      if (__any(hs[1] > SUM_LIMIT)) rescue(1, lastc);
      pv(std::integral_constant<int, 1>{});
    }
    l_run += hs[0] + hs[1];
    seen = true;
  };
  for (int tile = 0; tile + 1 < ntiles; ++tile) tile_body(tile, std::false_type{});
  tile_body(ntiles - 1, std::true_type{});

  if constexpr (SPLIT) {
    // Merge: every wave of a unit but its first (part 0) leaves O, m_ref and l (per lane) in the LDS ring, free once
    // every wave has passed its last tile; a wave that computed no tile (its keys all lie past L) leaves m = -inf.
    constexpr int SHARE = SPLIT == 2 ? WAVES : 2;  // waves per unit
    const int part = SPLIT == 2 ? wave : kh_sel;
    float* comb = reinterpret_cast<float*>(smem) + unit * (SHARE - 1) * MERGE_WORDS * 64 + lane;
    __syncthreads();
    if (active && part != 0) {
      float* mine = comb + (part - 1) * MERGE_WORDS * 64;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mine[(dt * 16 + r) * 64] = o[dt][r];
      mine[32 * 64] = seen ? m_ref : -__builtin_inff();
      mine[33 * 64] = l_run;
    }
    __syncthreads();
    if (!active || part != 0) return;
    float m = m_ref;
#pragma unroll
    for (int k = 1; k < SHARE; ++k) m = fmaxf(m, comb[((k - 1) * MERGE_WORDS + 32) * 64]);
    const float c0 = __builtin_amdgcn_exp2f(m_ref - m);
    l_run = l_run * c0;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] = o[dt][r] * c0;
#pragma unroll
    for (int k = 1; k < SHARE; ++k) {
      const float* theirs = comb + (k - 1) * MERGE_WORDS * 64;
      const float ck = __builtin_amdgcn_exp2f(theirs[32 * 64] - m);
      l_run = l_run + theirs[33 * 64] * ck;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = o[dt][r] + theirs[(dt * 16 + r) * 64] * ck;
    }
  } else {
    if (!active) return;
  }

  const float l_tot = l_run + xor_shuffle(l_run, 32);
  const float inv = 1.f / l_tot;
  const int q = q0 + fr;
  if (q < L) {
    half_t* orow = out + (tok0 + q) * C + h * HD;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        half4_t v;
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = static_cast<half_t>(o[dt][4 * g + u] * inv);
        *reinterpret_cast<half4_t*>(orow + dt * 32 + 8 * g + 4 * fh) = v;
      }
  }
}

// bq: queries per workgroup, BQ (one 32-query unit per wave) or BQ / 2 (two units, each over two waves by key half:
// twice the workgroups for grids far from filling the GPU once).
__global__ __launch_bounds__(64 * WAVES, 4) void attention_kernel(const half_t* __restrict__ qkv,
                                                                  half_t* __restrict__ out, int L, int H, int bq) {
  // K tile of ring slot st at smem + st*TILE, V tile at smem + (STAGES + st)*TILE
  __shared__ __attribute__((aligned(1024))) half_t smem[2 * STAGES * TILE];
  // 1-D grid over (sequence, head, query block), query block fastest, remapped so that all query blocks of one
  // (sequence, head) run on one XCD and read its K and V through one L2. When each XCD's share is whole (sequence,
  // head) groups, its partial last query blocks (L = 1025: a single query, a quarter of a block's time) are ordered
  // after its whole blocks, so they fill the end of the grid instead of leaving it to a last round of whole blocks
  // (measured at 32 x 16 x 1025: 169.4 vs 172.6 us; at 16 x 16 x 1025: 87.8 vs 91.0; the same results).
  const int nq = (L + bq - 1) / bq;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  int qb = t % nq, h = (t / nq) % H, seq = t / (nq * H);
  const int per = static_cast<int>(gridDim.x) >> 3;  // blocks per XCD
  if ((gridDim.x & 7) == 0 && per % nq == 0 && L % bq != 0 && nq > 1) {
    const int x = t / per, k = t % per, whole = per / nq * (nq - 1);
    const int pair = x * (per / nq) + (k < whole ? k / (nq - 1) : k - whole);
    qb = k < whole ? k % (nq - 1) : nq - 1;
    h = pair % H;
    seq = pair / H;
  }
  const int q_first = qb * bq;
  const int units = min(bq / QW, (L - q_first + QW - 1) / QW);  // 32-query units of this block
  if (units == 1)
    attention_block<2>(qkv, out, L, H, q_first, h, seq, smem);
  else if (2 * units <= WAVES)
    attention_block<1>(qkv, out, L, H, q_first, h, seq, smem);
  else
    attention_block<0>(qkv, out, L, H, q_first, h, seq, smem);
}

}  // namespace ff

using namespace ff;

extern "C" int ff_attention(const void* qkv, void* out, int64_t T, int64_t heads, int64_t seq_len, void* stream) {
  clear_error();
  if (heads <= 0 || heads > 65535) return fail(FF_EINVAL, "attention: need 0 < heads <= 65535");
  if (seq_len <= 0 || seq_len > 0x7fffffff) return fail(FF_EINVAL, "attention: need seq_len > 0");
  if (T < 0 || T % seq_len != 0) return fail(FF_EINVAL, "attention: T must be a multiple of seq_len");
  // K/V tiles are addressed by 32-bit byte offsets within one sequence
  if (seq_len * heads * 3 * HD * 2 >= (int64_t(1) << 31)) return fail(FF_EINVAL, "attention: sequence too large");
  const int64_t seqs = T / seq_len;
  if (T == 0) return FF_OK;
  if (!qkv || !out) return fail(FF_EINVAL, "attention: null pointer");
  if ((reinterpret_cast<uintptr_t>(qkv) & 15) || (reinterpret_cast<uintptr_t>(out) & 7))
    return fail(FF_EINVAL, "attention: misaligned pointer");
  // 128-query blocks; 64-query blocks (twice as many) when those still fit the GPU's resident workgroups at once.
  // Measured: EVA02-L at batch 1 (144 -> 288 blocks) 16.4 -> 15.1 us; grids that the halving pushes past one round
  // run slower (PixAI's windows, 720 -> 1296 blocks: 23.9 -> 27.3 us), and so did 32-query blocks at batch 1.
  int64_t resident = resident_blocks(reinterpret_cast<const void*>(&attention_kernel), 64 * WAVES, 0);
  if (resident <= 0) resident = 1024;
  const int bq = (seq_len + BQ / 2 - 1) / (BQ / 2) * heads * seqs <= resident ? BQ / 2 : BQ;
  const int64_t blocks = (seq_len + bq - 1) / bq * heads * seqs;
  if (blocks > 0x7fffffff) return fail(FF_EINVAL, "attention: too many blocks");
  const dim3 grid(static_cast<unsigned>(blocks));
  attention_kernel<<<grid, 64 * WAVES, 0, as_stream(stream)>>>(static_cast<const half_t*>(qkv),
                                                                static_cast<half_t*>(out), static_cast<int>(seq_len),
                                                                static_cast<int>(heads), bq);
  return check_launch("attention");
}
