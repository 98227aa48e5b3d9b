// Tile helpers shared by the workgroup-cooperative kernels (bf16, gfx950):
// 32-edge tiles as two 16-column MFMA blocks, chain-ordered LDS buffers that
// pass one stage's C-blocks to the next stage as B operands, identity-MFMA
// transposes to edge-major operands, and the 0/1 segment matrix of the per-row
// sums.  See egnn_device.h for the operand model.
#pragma once
#include "egnn_device.h"
#include "egnn_internal.h"

namespace egnn {
namespace tile {

constexpr int TE = kTileEdges;  // 32 edges = two 16-column MFMA blocks

__device__ __forceinline__ bf16x4 pack4(const f32x4& v) {
  bf16x4 r;
  r[0] = (bf16)v[0]; r[1] = (bf16)v[1]; r[2] = (bf16)v[2]; r[3] = (bf16)v[3];
  return r;
}
__device__ __forceinline__ f32x4 unpack4(const bf16x4& v) {
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// chain buffer over NB 16-edge blocks: chunk (kc, nb) = 64 lanes x 8 bf16 at index kc NB + nb;
// 16-row block blk fills half (blk & 1) of chunk blk >> 1.  With SW the 16-byte lane slot s of a
// chunk is stored at s ^ 4 ((s >> 4) & 3) (within its aligned group of 16 slots): the 8-byte
// transposing reads of chain_edge_major (lanes of g = 0, 1 read slots 16 q + 4 g + b, q = c & 3,
// b = c >> 2) then fall on 16 different slots mod 16, two lanes each, instead of 8 slots, four
// lanes each; the lane-order reads and writes keep their bank spread.
template <bool SW>
__device__ __forceinline__ int chain_slot(int s) { return SW ? s ^ (((s >> 4) & 3) << 2) : s; }
template <int NB = 2, bool SW = false>
__device__ __forceinline__ void put_chain(bf16* buf, int blk, int nb, int l, const f32x4& v) {
  *reinterpret_cast<bf16x4*>(buf + (((blk >> 1) * NB + nb) * 64 + chain_slot<SW>(l)) * 8 + 4 * (blk & 1)) = pack4(v);
}
template <int NB = 2, bool SW = false>
__device__ __forceinline__ bf16x8 get_chain(const bf16* buf, int kc, int nb, int l) {
  return *reinterpret_cast<const bf16x8*>(buf + ((kc * NB + nb) * 64 + chain_slot<SW>(l)) * 8);
}
// edge-major buffer: feature block blk, lane (c = feature, g) holds 8 edges in kappa_chain order
__device__ __forceinline__ void put_norm(bf16* buf, int blk, int l, const bf16x8& v) {
  *reinterpret_cast<bf16x8*>(buf + (blk * 64 + l) * 8) = v;
}
__device__ __forceinline__ bf16x8 get_norm(const bf16* buf, int blk, int l) {
  return *reinterpret_cast<const bf16x8*>(buf + (blk * 64 + l) * 8);
}

// B operand that transposes one 16-row C-block: B[s][n] = (s < 4 && 4g + s == n)
__device__ __forceinline__ bf16x8 ident_chunk(int c, int g) {
  bf16x8 r = zero_chunk<bf16>();
  const int s = c - 4 * g;
#pragma unroll
  for (int q = 0; q < 4; ++q) r[q] = (s == q) ? (bf16)1.0f : (bf16)0.0f;
  return r;
}
// C-block (rows = 16 features, col = edge c) -> C-block (col = feature c, rows = edges 4g+i), bf16-rounded
__device__ __forceinline__ f32x4 transpose_block(const f32x4& v, const bf16x8& I) {
  bf16x8 a = zero_chunk<bf16>();
  a[0] = (bf16)v[0]; a[1] = (bf16)v[1]; a[2] = (bf16)v[2]; a[3] = (bf16)v[3];
  f32x4 t = zero4();
  mma(t, a, I);
  return t;
}
// edge-major chunk of a feature block over the 32 edges of the tile (kappa_chain over edges)
__device__ __forceinline__ bf16x8 edge_major(const f32x4& nb0, const f32x4& nb1, const bf16x8& I) {
  return pack_chunk<bf16>(transpose_block(nb0, I), transpose_block(nb1, I));
}
// The same chunk for 16-row block blk read back from a chain buffer that holds it
// (put_chain of the edge blocks 2 eh, 2 eh + 1: edges 32 eh .. 32 eh + 31), by two transposing
// reads.  Feature 16 (blk & 1) + 4q + i of group blk >> 1 and edge e sit at lane slot
// 16q + (e & 15) of chunk (blk >> 1, e >> 4), element 4 (blk & 1) + i.  Within a 16-lane group,
// lane j addresses edge kb + j/4, features 4 (j % 4) .. + 3, and lane c receives
// feature c of edges kb .. kb + 3: kb = 4g gives elements 0..3, kb = 16 + 4g 4..7.
template <int NB = 2, bool SW = false>
__device__ __forceinline__ bf16x8 chain_edge_major(const bf16* buf, int blk, int c, int g, int eh = 0) {
  const bf16* base = buf + ((blk >> 1) * NB + 2 * eh) * 64 * 8 + 4 * (blk & 1);
  const int e0 = 4 * g + (c >> 2);         // edges of the first read: 0..15, block 0
  const int sl = chain_slot<SW>(16 * (c & 3) + e0);
  const bf16* p0 = base + sl * 8;
  const bf16* p1 = base + (64 + sl) * 8;   // edge 16 + e0: chunk of edge block 1, lane slot 16q + e0
  const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)p0);
  const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)p1);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Edge-feature tile stored slot-major for the dW_e products: row `slot` holds the tile's 32
// edges in kappa_chain order, so the B operand of lane (c, g) (edges kappa_chain(g, s) of one
// slot) is one 16-byte read.  Edge 16 nb + c sits at position 8 (c >> 2) + 4 nb + (c & 3).
__device__ __forceinline__ void put_ut(bf16* buf, int nb, int c, int g, const bf16x8& u) {
  bf16* p = buf + 8 * g * TE + 8 * (c >> 2) + 4 * nb + (c & 3);   // slots 8g .. 8g + 7 of the edge
#pragma unroll
  for (int s = 0; s < 8; ++s) p[s * TE] = u[s];
}
__device__ __forceinline__ bf16x8 get_ut(const bf16* buf, int slot, int g) {
  return *reinterpret_cast<const bf16x8*>(buf + slot * TE + 8 * g);
}
// The A chunk over the tile's 32 edges (kappa_chain) of a C-block transposed to edge-major
// (transpose_block) that covers only edge block nb: elements 4 nb .. 4 nb + 3, zeros elsewhere.
// nb must be wave-uniform (a select of whole registers, no per-element moves).
__device__ __forceinline__ bf16x8 half_edge_chunk(const f32x4& t, int nb) {
  const u32x2 v = __builtin_bit_cast(u32x2, pack4(t));
  const u32x4 q = nb ? u32x4{0u, 0u, v[0], v[1]} : u32x4{v[0], v[1], 0u, 0u};
  return __builtin_bit_cast(bf16x8, q);
}

__device__ __forceinline__ int rank_of(uint32_t mask, int k) {
  const uint32_t below = (k >= 31) ? 0xffffffffu : ((2u << k) - 1u);
  return __popc(mask & below) - 1;
}
// B operand S[edge][rank]: column n = rank 16*rb + c, rows = edges kappa_chain(g, s)
__device__ __forceinline__ bf16x8 seg_chunk(uint32_t mask, int nvalid, int rb, int c, int g) {
  bf16x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int k = kappa_chain(g, s);
    r[s] = (k < nvalid && rank_of(mask, k) == 16 * rb + c) ? (bf16)1.0f : (bf16)0.0f;
  }
  return r;
}

// A operand that adds two 4-row halves of a B chunk: A[r][8g + s] = (r == 4g + (s & 3)), so
// the product with B = [P rows 4g..4g+3 | Q rows 4g..4g+3] (lane g) is P + Q on rows 4g..4g+3
__device__ __forceinline__ bf16x8 pair_sum_chunk(int c, int g) {
  bf16x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) r[s] = (c - 4 * g == (s & 3)) ? (bf16)1.0f : (bf16)0.0f;
  return r;
}

// P_i + Q_j of a 16-feature block from one gathered B chunk: lanes g = 0, 1 of
// edge column c hold P features 8g .. 8g + 7 of the block, lanes g = 2, 3 Q
// features 8(g - 2) .. + 7 (pq_gather); A[r][k] = 1 where k is P or Q feature r.
__device__ __forceinline__ bf16x8 pq_sum_chunk(int c, int g) {
  bf16x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) r[s] = ((g & 1) == (c >> 3) && s == (c & 7)) ? (bf16)1.0f : (bf16)0.0f;
  return r;
}
// The B chunk of pq_sum_chunk for feature block blk: one 16-byte load per lane from
// the natural-order P | Q rows (4H bytes each) of row i (P) or source j (Q).
__device__ __forceinline__ bf16x8 pq_gather(const char* PQb, uint32_t i, uint32_t j, int blk, int g, int H) {
  const uint32_t row = g < 2 ? i : j;
  const uint32_t off = 2u * (uint32_t)((g < 2 ? 0 : H) + 16 * blk + 8 * (g & 1));
  return *reinterpret_cast<const bf16x8*>(PQb + (row * (4u * (uint32_t)H) + off));
}

// 16 bf16x4 patterns: element s of entry n is 1.0 when bit s of n is set
__device__ __forceinline__ void seg_lut_init(uint2* lut, int tid) {
  if (tid < 16) {
    const uint32_t one = 0x3F80u;
    lut[tid] = make_uint2(((tid & 1) ? one : 0u) | ((tid & 2) ? one << 16 : 0u),
                          ((tid & 4) ? one : 0u) | ((tid & 8) ? one << 16 : 0u));
  }
}
// Span of a rank within the tile: first edge (bits 0-7) and edge count (bits 8-15).
__device__ __forceinline__ int rank_span(int start, int count) { return start | (count << 8); }
// B operand S[edge][rank] from the span of rank 16 rb + c (0 when there is no such rank):
// lane (c, g) covers edges kappa_chain(g, s) = 4g..4g+3 and 16+4g..16+4g+3
__device__ __forceinline__ bf16x8 seg_chunk_span(int span, int g, const uint2* lut) {
  const int start = span & 0xff, cnt = span >> 8;
  const uint32_t mrow = cnt >= 32 ? 0xffffffffu : (((1u << cnt) - 1u) << start);
  const uint2 lo = lut[(mrow >> (4 * g)) & 15u];
  const uint2 hi = lut[(mrow >> (16 + 4 * g)) & 15u];
  bf16x8 r;
  const uint4 v = make_uint4(lo.x, lo.y, hi.x, hi.y);
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// B operand S[edge][rank] of the rank with this span (0: no rank), made with vector instructions:
// lane (c, g) covers edges 4g..4g+3 and 16+4g..16+4g+3 (the pattern of seg_chunk_span, without its table)
__device__ __forceinline__ bf16x8 seg_chunk_valu(int span, int g) {
  const int start = span & 0xff, cnt = span >> 8;
  const uint32_t mrow = cnt >= 32 ? 0xffffffffu : (((1u << cnt) - 1u) << start);
  const uint32_t x = (mrow >> (4 * g)) & 15u, y = (mrow >> (16 + 4 * g)) & 15u;
  auto pat = [](uint32_t b) { return ((b & 1u) | ((b & 2u) << 15)) * 0x3F80u; };   // 1.0 in the set halves
  const uint4 v = make_uint4(pat(x), pat(x >> 2), pat(y), pat(y >> 2));
  bf16x8 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// Ranks of a 32-edge tile from the rows of its edges (ri[0..TE)) and of the edges
// just before and after it (ex[0], ex[1]): edge k starts a rank when it is the
// tile's first edge or its row differs from that of edge k - 1; the first rank's
// row starts in the tile unless edge base - 1 has the same row, the last rank's
// row ends in it unless edge base + TE has the same row.  Wave-uniform results.
struct TileRanks { uint32_t mask; int nrank, nvalid; bool start_in, end_in; };
__device__ __forceinline__ TileRanks tile_ranks(const int* ri, const int* ex, int64_t base, int64_t E, int l) {
  TileRanks r;
  r.nvalid = (int)((E - base) < TE ? (E - base) : TE);
  const int k = l & 31;
  const int rk = ri[k], rp = ri[k > 0 ? k - 1 : 0];
  const bool nf = l < TE && k < r.nvalid && (k == 0 || rp != rk);
  r.mask = (uint32_t)(__ballot(nf) & 0xffffffffull);
  r.nrank = __popc(r.mask);
  r.start_in = base == 0 || ex[0] != ri[0];
  r.end_in = base + TE >= E || ex[1] != ri[TE - 1];
  return r;
}
// Row and span of each rank (call from one wave): lane l < TE that starts rank q writes
// rowof[q] and rspan[q].
__device__ __forceinline__ void tile_rank_tables(const int* ri, const TileRanks& r, int l, int* rowof, int* rspan) {
  if (l < TE && ((r.mask >> l) & 1u)) {
    const uint32_t rest = l >= 31 ? 0u : (r.mask & ~((2u << l) - 1u));
    const int end = rest ? __ffs(rest) - 1 : r.nvalid;
    const int q = rank_of(r.mask, l);
    rowof[q] = ri[l];
    rspan[q] = rank_span(l, end - l);
  }
}
// Rank r of the tile is a whole row: it neither continues from the previous tile nor into the next.
__device__ __forceinline__ bool rank_whole(const TileRanks& rk, int r) {
  return (r > 0 || rk.start_in) && (r < rk.nrank - 1 || rk.end_in);
}

__device__ __forceinline__ bf16x8 input_chunk(const bf16* ef, int64_t se, int eid, int FE, int g, float r2, bool eq) {
  const int slot0 = 8 * g;
  if (slot0 + 8 <= FE) return load_chunk(ef + (int64_t)eid * se + slot0);
  bf16x8 z = zero_chunk<bf16>();
  if (eq && slot0 == FE) {
    const bf16 hi = (bf16)r2;
    z[0] = hi;
    z[1] = (bf16)(r2 - (float)hi);
  }
  return z;
}

__device__ __forceinline__ uint32_t lo16(unsigned long long b) { return (uint32_t)(b & 0xffffull); }

// A operands from a row-major bf16 matrix W in LDS (row pitch P), K slice kc,
// lane (c, g) element s <-> k = 32 kc + kappa_chain(g, s):
//   lds_rows: A[r][k] = W[r][k] for rows r = 16 blk + c (two 8-byte reads)
//   lds_cols: A[r][k] = W[k][r] (two transposing reads: within a 16-lane group,
//             lane j addresses row kb + j/4, columns 16 blk + 4 (j % 4) .. + 3,
//             and lane c receives column 16 blk + c of rows kb .. kb + 3)
template <int P>
__device__ __forceinline__ bf16x8 lds_rows(const bf16* W, int blk, int kc, int c, int g) {
  const bf16* p = W + (16 * blk + c) * P + 32 * kc + 4 * g;
  return __builtin_shufflevector(*reinterpret_cast<const bf16x4*>(p), *reinterpret_cast<const bf16x4*>(p + 16),
                                 0, 1, 2, 3, 4, 5, 6, 7);
}
template <int P>
__device__ __forceinline__ bf16x8 lds_cols(const bf16* W, int blk, int kc, int c, int g) {
  const bf16* p0 = W + (32 * kc + 4 * g + (c >> 2)) * P + 16 * blk + 4 * (c & 3);
  const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)p0);
  const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)(p0 + 16 * P));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// dst[i][j] (DR x DC, row pitch P) = W[i][j] from W^T (DC x DR) row-major: one
// 8 x 8 block per thread, transposed in registers, 16-byte reads and writes
template <int DR, int DC, int P, int NT>
__device__ __forceinline__ void fill_weight_lds_t(bf16* dst, const bf16* src) {
  for (int q = threadIdx.x; q < (DR / 8) * (DC / 8); q += NT) {
    const int ib = q % (DR / 8), jb = q / (DR / 8);   // rows 8 ib .. + 7, columns 8 jb .. + 7 of W
    bf16x8 v[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) v[r] = load_chunk(src + (int64_t)(8 * jb + r) * DR + 8 * ib);   // v[r][u] = W[8 ib + u][8 jb + r]
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      bf16x8 o;
#pragma unroll
      for (int r = 0; r < 8; ++r) o[r] = v[r][u];
      *reinterpret_cast<bf16x8*>(dst + (8 * ib + u) * P + 8 * jb) = o;
    }
  }
}

// dst[i][j] (DR x DC, row pitch P) = W[i][j] of a row-major weight matrix;
// block-cooperative 16-byte reads and writes
template <int DR, int DC, int P, int NT>
__device__ __forceinline__ void fill_weight_lds(bf16* dst, const bf16* src) {
  for (int q = threadIdx.x; q < DR * DC / 8; q += NT) {
    const int i = q / (DC / 8), j = 8 * (q % (DC / 8));
    *reinterpret_cast<bf16x8*>(dst + i * P + j) = load_chunk(src + (int64_t)i * DC + j);
  }
}

// A 128 x 128 weight W[r][k] in LDS as rows of 144 bf16 (288 bytes), the 8-byte unit u of row R stored at
// unit u ^ ((R >> 2) & 3).  Both operand reads then hit 16 different 8-byte bank groups per 16 lanes: the
// row reads of W (lanes c read rows 16 blk + c at one unit) and the transposing reads of W^T (lanes read
// rows kb + c / 4 at units 4 blk + c % 4).  The swizzle changes only the two low bits
// of a unit, so every fragment's address is a per-lane base plus a constant.
constexpr int kWP = 144;
__device__ __forceinline__ const bf16* wunit(const bf16* W, int R, int u) { return W + R * kWP + 4 * (u ^ ((R >> 2) & 3)); }
// A[r][k] = W[16 blk + r][32 kc + kappa_chain(g, s)]  (S5: A = W_hl); Wr = the lane's base, wrow_base
__device__ __forceinline__ const bf16* wrow_base(const bf16* W, int c, int g) { return W + c * kWP + 4 * (g ^ ((c >> 2) & 3)); }
__device__ __forceinline__ bf16x8 w_rows(const bf16* Wr, int blk, int kc) {
  const bf16* p = Wr + 16 * blk * kWP + 32 * kc;
  return __builtin_shufflevector(*reinterpret_cast<const bf16x4*>(p), *reinterpret_cast<const bf16x4*>(p + 16),
                                 0, 1, 2, 3, 4, 5, 6, 7);
}
// A[r][k] = W[32 kc + kappa_chain(g, s)][16 blk + r]  (S2: A = W_hl^T), two transposing reads: lane c
// addresses row kb + c / 4, columns 16 blk + 4 (c % 4) .. + 3, and receives column 16 blk + c of rows
// kb .. kb + 3; Wc = the lane's base, wcol_base
__device__ __forceinline__ const bf16* wcol_base(const bf16* W, int c, int g) {
  return W + (4 * g + (c >> 2)) * kWP + 4 * ((c & 3) ^ (g & 3));
}
__device__ __forceinline__ bf16x8 w_cols(const bf16* Wc, int blk, int kc) {
  const bf16* p = Wc + 32 * kc * kWP + 16 * blk;
  const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)p);
  const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)(p + 16 * kWP));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// W (R x C) into the swizzled rows, one 8-byte unit per step, from W given row-major (src[r][c]) or as its
// transpose (lin: src[c][r])
template <int R, int C, int NT>
__device__ __forceinline__ void fill_weight_swizzled(bf16* dst, const bf16* src, bool lin) {
  for (int q = threadIdx.x; q < R * C / 4; q += NT) {
    const int r = q / (C / 4), u = q % (C / 4);
    bf16x4 v;
    if (lin) {
#pragma unroll
      for (int t = 0; t < 4; ++t) v[t] = src[(int64_t)(4 * u + t) * R + r];
    } else {
      v = *reinterpret_cast<const bf16x4*>(src + (int64_t)r * C + 4 * u);
    }
    *reinterpret_cast<bf16x4*>(const_cast<bf16*>(wunit(dst, r, u))) = v;
  }
}

}  // namespace tile
}  // namespace egnn
