// gemm_tiled.hip -- the a9 Q8_0 x Q8_0 and a7 Q4_0 x Q8_0 GEMMs over operands
// in the GEMM-tile layout, staged into LDS by DMA (buffer_load_dwordx4 ... lds,
// global_load_lds_dwordx4): no staging registers and no staging VALU, so every
// VGPR and VALU cycle goes to the fold.  Two work-group tiles: 256 weight rows
// x 128 tokens (16 waves of 2 tiles, gemm_tiles_q8 / gemm_tiles_q4) and 256 x
// 256 (8 waves of 2 x 4 tiles, gemm_tiles256_q8 / gemm_tiles256_q4); the
// entries pick per shape (tiles256_first), the results are the same bits.
//
// GEMM-tile layout of a Q8_0 matrix of nrows rows x nb blocks (the same bytes
// as the plain rows, regrouped): rows in groups of 64; for group g and block b
// one 2176-byte record at (g*nb + b)*2176:
//   bytes    0..1023  quants 0..15 of the block for rows 64g+0..63, 16 B a row
//   bytes 1024..2047  quants 16..31, the same way
//   bytes 2048..2175  the 64 fp16 scales
// Rows past nrows in the last group are zero.  A record's halves are the
// operand of one v_mfma_i32_32x32x32_i8 lane (16 quants), already 16-byte
// aligned, so a wave moves one half of 64 rows with one 1 KB DMA instruction.
//
// Q4_0 weights take the same records with each nibble decoded to its signed
// quant q - 8 (element j < 16 from the low nibble of quant byte j, 16 + j from
// its high nibble) and the fp16 scale copied.
//
// Semantics are those of tcrv_hip_q8_0_q8_0_gemm and tcrv_hip_q4_0_q8_0_gemm
// (gemm.hip): every output is the a5 / a6 block dot, folded in ascending block
// order (mfma_fold.h).
#include "mfma_fold.h"

namespace tcrv {

constexpr int kTG = 64;                        // rows per tile group
constexpr int kTRec = 2 * kTG * 16 + kTG * 2;  // 2176 bytes per (group, block) record
// The 256 x 128 kernels' K chunk and LDS stages, 4096^3 on one box (us): 6 blocks
// x 2 stages 163.7-164.4, 5 x 2 163.5, 4 x 3 169.7-170.5, 3 x 3 174.9: one chunk
// in flight covers the DMA latency, and longer chunks meet at fewer barriers.
constexpr int kDBM = 256, kDBN = 128, kDKB = 6;  // work-group tile, blocks per K chunk
constexpr int kDRows = kDBM + kDBN;               // 384 staged rows
constexpr int kDHalf = kDRows * 16;               // 6144: one half of one block, all rows
constexpr int kDBlock = 2 * kDHalf;               // 12288: both halves of one block
constexpr int kDStage = kDKB * kDBlock;           // 73728 quant bytes per stage
constexpr int kDHRow = kDRows + 32;               // fp16 scales per block row (+32 zero rows)
constexpr int kDThreads = 1024;
constexpr int kDQuantDma = kDKB * 2 * (kDRows / kTG);  // 72 quant DMA instructions per chunk
constexpr int kDDma = kDQuantDma + kDKB;               // + one scale instruction per block
constexpr int kDStages = 2;  // chunks c+1 .. c+kDStages-1 in flight while chunk c is
                             // folded (2 or 3)
constexpr int kDSlots = (kDDma + 15) / 16;   // DMA instructions per wave and chunk
static_assert(kDStages == 2 || kDStages == 3, "prefetch distance 1 or 2");
// the Q4_0 kernel also keeps its token scales widened to fp32: kDBN per block
static_assert(kDStages * (kDKB * 12288 + kDKB * (kDBM + kDBN + 32) * 2 + kDKB * kDBN * 4) <=
                  160 * 1024,
              "the stages fit the 160 KB of LDS");

// ---------------------------------------------------------------- pack ---
// Rows 16-byte aligned (and bx % 16 == 0): one wave per (group, 8-block range),
// lane r = row 64g + r.  Blocks 8c..8c+7 of a row are 272 contiguous bytes at a
// 16-byte aligned offset (8 x 34 = 17 x 16), so the lane loads them with 17
// 128-bit loads, all issued before the first use, and the whole span of the
// row's cache lines is read by one wave (a wave per record read each line from
// up to three XCDs).  The eight records are then written from registers, every
// store 64 consecutive 16-byte (or 2-byte) slots.
constexpr int kPackSpan = 8;  // blocks per lane (4096 rows x 128 blocks: 7.3 us; the
                              // per-record kernel 9.3 us; two waves per 8-block span
                              // with 9 loads each 12.2 us)

// Lane r's part of one record: its row's 32 quants (two 16-byte slots of the
// record's 64-slot halves) and its fp16 scale.  kStream: nontemporal stores,
// for a pack whose output is not read right away (4096 rows x 128 blocks, 24
// rotating operands past the Infinity Cache, interleaved runs: Q8_0 8.13
// against 9.79 us, Q4_0 5.31 against 7.56 us).
// The packs inside one GEMM call keep ordinary stores: the GEMM that follows
// reads the records from the caches (Q4_0 4096^3 ws entry: 224.6 against
// 210.5 us with streaming stores).
template <bool kStream>
__device__ __forceinline__ void store_record(uint8_t *o, int r, const uint32_t (&q)[8],
                                             uint32_t d) {
  if constexpr (kStream) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 lo = {q[0], q[1], q[2], q[3]}, hi = {q[4], q[5], q[6], q[7]};
    __builtin_nontemporal_store(lo, reinterpret_cast<u32x4 *>(o) + r);
    __builtin_nontemporal_store(hi, reinterpret_cast<u32x4 *>(o + 1024) + r);
    __builtin_nontemporal_store(static_cast<uint16_t>(d), reinterpret_cast<uint16_t *>(o + 2048) + r);
  } else {
    reinterpret_cast<uint4 *>(o)[r] = make_uint4(q[0], q[1], q[2], q[3]);
    reinterpret_cast<uint4 *>(o + 1024)[r] = make_uint4(q[4], q[5], q[6], q[7]);
    reinterpret_cast<uint16_t *>(o + 2048)[r] = static_cast<uint16_t>(d);
  }
}

// Span `wave` of one operand (64-row group g, 8-block span c), lane r = row
// 64g + r.
template <bool kStream>
__device__ __forceinline__ void pack_span(size_t nrows, size_t nb, const uint8_t *src,
                                          size_t bx, uint8_t *dst, size_t wave, int r) {
  const size_t spans_per_group = nb / kPackSpan;
  const size_t g = wave / spans_per_group, c = wave - g * spans_per_group;
  const size_t row = g * kTG + r;
  uint32_t v[4 * 17];
  if (row < nrows) {
    const uint4 *p = reinterpret_cast<const uint4 *>(src + row * bx + c * kPackSpan * kQ8Bytes);
#pragma unroll
    for (int k = 0; k < 17; ++k) {
      const uint4 x = p[k];
      v[4 * k] = x.x; v[4 * k + 1] = x.y; v[4 * k + 2] = x.z; v[4 * k + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 68; ++k)
      v[k] = 0;  // rows past nrows in the last group are zero
  }
#pragma unroll
  for (int k = 0; k < kPackSpan; ++k) {
    // block k at byte 34k of the span: even k -> dword 17k/2 holds the scale in
    // its low half and the quants start 2 bytes in; odd k -> the scale is the
    // high half of dword (34k-2)/4 and the quants are the next 8 dwords
    uint32_t q[8], d;
    if ((k & 1) == 0) {
      const int w0 = 17 * k / 2;
      d = v[w0] & 0xffffu;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        q[j] = funnel16(v[w0 + j], v[w0 + j + 1]);
    } else {
      const int w0 = (34 * k - 2) / 4;
      d = v[w0] >> 16;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        q[j] = v[w0 + 1 + j];
    }
    store_record<kStream>(dst + (g * nb + c * kPackSpan + k) * kTRec, r, q, d);
  }
}

__global__ __launch_bounds__(256) void pack_gemm_tiles_span(size_t nrows, size_t nb,
                                                            const uint8_t *src, size_t bx,
                                                            uint8_t *dst, size_t nspans) {
  const size_t wave = (static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
  if (wave >= nspans)
    return;
  pack_span<true>(nrows, nb, src, bx, dst, wave, static_cast<int>(threadIdx.x & 63));
}

// One wave per (group, block) record for blocks b0.. of every group, lane
// r = row 64g + r.  kAligned: the rows are 4-byte aligned (dword loads,
// realigned with v_alignbyte for even blocks); otherwise 16-bit loads.
template <bool kAligned>
__global__ __launch_bounds__(256) void pack_gemm_tiles(size_t nrows, size_t nb,
                                                       const uint8_t *src, size_t bx,
                                                       uint8_t *dst, size_t b0, size_t nrec) {
  const size_t t = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  const size_t rec = t >> 6;
  if (rec >= nrec)
    return;
  const int r = static_cast<int>(t & 63);
  const size_t per_group = nb - b0;
  const size_t g = rec / per_group, b = b0 + (rec - g * per_group);
  const size_t row = g * kTG + r;
  uint32_t q[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  uint32_t d = 0;
  if (row < nrows) {
    const uint8_t *blk = src + row * bx + b * kQ8Bytes;
    if constexpr (kAligned) {
      if ((b & 1) == 0) {  // block 4-byte aligned: scale, then quants at +2
        const uint32_t *w = reinterpret_cast<const uint32_t *>(blk);
        uint32_t v[9];
#pragma unroll
        for (int k = 0; k < 8; ++k)
          v[k] = w[k];
        v[8] = *reinterpret_cast<const uint16_t *>(blk + 32);
        d = v[0] & 0xffffu;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          q[k] = funnel16(v[k], v[k + 1]);
      } else {  // quants 4-byte aligned, the scale in the dword before them
        const uint32_t *w = reinterpret_cast<const uint32_t *>(blk - 2);
        d = w[0] >> 16;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          q[k] = w[k + 1];
      }
    } else {
      const uint16_t *h = reinterpret_cast<const uint16_t *>(blk);
      d = h[0];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        q[k] = static_cast<uint32_t>(h[1 + 2 * k]) | (static_cast<uint32_t>(h[2 + 2 * k]) << 16);
    }
  }
  uint8_t *o = dst + (g * nb + b) * kTRec;
  reinterpret_cast<uint4 *>(o)[r] = make_uint4(q[0], q[1], q[2], q[3]);
  reinterpret_cast<uint4 *>(o + 1024)[r] = make_uint4(q[4], q[5], q[6], q[7]);
  reinterpret_cast<uint16_t *>(o + 2048)[r] = static_cast<uint16_t>(d);
}

// Q4_0 rows into the same layout with every nibble decoded to the int8 it
// stands for (n - 8): quants 0-15 are the low nibbles of the 16 quant bytes,
// 16-31 the high nibbles.  The subtraction is bytewise and carry-free:
// n + 0x78 stays below 0x100, and flipping bit 7 maps it to n - 8.
__device__ __forceinline__ void decode_q4_quants(const uint32_t w[4], uint32_t q[8]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    q[m] = ((w[m] & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
    q[4 + m] = (((w[m] >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
  }
}

// Span `wave` of one Q4_0 operand with 16-byte aligned rows (bx % 16 == 0):
// 64-row group g, 8-block span c, lane r = row 64g + r; the span is 144
// contiguous bytes (9 aligned 128-bit loads), block k at byte 18k.
template <bool kStream>
__device__ __forceinline__ void pack_q4_span(size_t nrows, size_t nb, const uint8_t *src,
                                             size_t bx, uint8_t *dst, size_t wave, int r) {
  const size_t spans_per_group = nb / kPackSpan;
  const size_t g = wave / spans_per_group, c = wave - g * spans_per_group;
  const size_t row = g * kTG + r;
  uint32_t v[4 * 9];
  if (row < nrows) {
    const uint4 *p = reinterpret_cast<const uint4 *>(src + row * bx + c * kPackSpan * kQ4Bytes);
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      const uint4 x = p[k];
      v[4 * k] = x.x; v[4 * k + 1] = x.y; v[4 * k + 2] = x.z; v[4 * k + 3] = x.w;
    }
  }
#pragma unroll
  for (int k = 0; k < kPackSpan; ++k) {
    // even k: the scale is the low half of dword 9k/2, the quants 2 bytes in;
    // odd k: the high half of dword (18k-2)/4, the quants the next 4 dwords
    uint32_t w[4] = {0, 0, 0, 0}, d = 0;
    if (row < nrows) {
      if ((k & 1) == 0) {
        const int w0 = 9 * k / 2;
        d = v[w0] & 0xffffu;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          w[j] = funnel16(v[w0 + j], v[w0 + j + 1]);
      } else {
        const int w0 = (18 * k - 2) / 4;
        d = v[w0] >> 16;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          w[j] = v[w0 + 1 + j];
      }
    }
    uint32_t q[8];
    decode_q4_quants(w, q);
    if (row >= nrows) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        q[j] = 0;  // rows past nrows in the last group are zero
    }
    store_record<kStream>(dst + (g * nb + c * kPackSpan + k) * kTRec, r, q, d);
  }
}

// One wave per (group, span) of one Q4_0 operand.
__global__ __launch_bounds__(256) void pack_q4_tiles_span(size_t nrows, size_t nb,
                                                          const uint8_t *src, size_t bx,
                                                          uint8_t *dst, size_t nspans) {
  const size_t wave = (static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
  if (wave >= nspans)
    return;
  pack_q4_span<true>(nrows, nb, src, bx, dst, wave, static_cast<int>(threadIdx.x & 63));
}

// One wave per (group, block) record for blocks b0.. of every group (rows
// 2-byte aligned: 16-bit loads).
__global__ __launch_bounds__(256) void pack_q4_tiles(size_t nrows, size_t nb, const uint8_t *src,
                                                     size_t bx, uint8_t *dst, size_t b0,
                                                     size_t nrec) {
  const size_t t = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  const size_t rec = t >> 6;
  if (rec >= nrec)
    return;
  const int r = static_cast<int>(t & 63);
  const size_t per_group = nb - b0;
  const size_t g = rec / per_group, b = b0 + (rec - g * per_group);
  const size_t row = g * kTG + r;
  uint32_t w[4] = {0, 0, 0, 0}, d = 0;
  if (row < nrows) {
    const uint16_t *hp = reinterpret_cast<const uint16_t *>(src + row * bx + b * kQ4Bytes);
    d = hp[0];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = static_cast<uint32_t>(hp[1 + 2 * j]) | (static_cast<uint32_t>(hp[2 + 2 * j]) << 16);
  }
  uint32_t q[8];
  decode_q4_quants(w, q);
  if (row >= nrows) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      q[j] = 0;
  }
  uint8_t *o = dst + (g * nb + b) * kTRec;
  reinterpret_cast<uint4 *>(o)[r] = make_uint4(q[0], q[1], q[2], q[3]);
  reinterpret_cast<uint4 *>(o + 1024)[r] = make_uint4(q[4], q[5], q[6], q[7]);
  reinterpret_cast<uint16_t *>(o + 2048)[r] = static_cast<uint16_t>(d);
}

// Both operands of one GEMM in one launch (their spans back to back in the
// grid): one launch instead of two, and twice the loads in flight.  kXQ4: the
// first operand is Q4_0 weights.
struct SpanOperand {
  const uint8_t *src;
  size_t bx, nrows, nspans;
  uint8_t *dst;
};

template <bool kXQ4>
__global__ __launch_bounds__(256) void pack_gemm_tiles_span2(size_t nb, SpanOperand x,
                                                             SpanOperand y) {
  size_t wave = (static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
  const int r = static_cast<int>(threadIdx.x & 63);
  if (wave < x.nspans) {
    if constexpr (kXQ4)
      pack_q4_span<false>(x.nrows, nb, x.src, x.bx, x.dst, wave, r);
    else
      pack_span<false>(x.nrows, nb, x.src, x.bx, x.dst, wave, r);
    return;
  }
  wave -= x.nspans;
  if (wave < y.nspans)
    pack_span<false>(y.nrows, nb, y.src, y.bx, y.dst, wave, r);
}

// ---------------------------------------------------------------- GEMM ---
typedef __attribute__((address_space(3))) void lds_void;

// The DMA of one K chunk is kDDma wave instructions: j < kDQuantDma moves
// half h of block b of one 64-row group (A groups 0-3, B groups 4-5) -- 1 KB,
// lane l its 16 bytes of row l; j >= kDQuantDma the scales of block
// j - kDQuantDma of all six groups (48 lanes, 16 bytes each).  Wave w issues
// j = w, w+16, w+32, ... (kDSlots of them): its "slots", whose sources (chunk
// 0) and LDS offsets (stage 0) are computed once; chunk c adds c*kDKB records,
// stage st a fixed offset.  Every slot but the last is a quant slot for every
// wave, so its source is a wave-uniform record half (scalar registers) plus
// the lane's 16-byte offset; the last slot, a scale slot on some waves, keeps
// a per-lane address.  Groups past the operand's last one re-read the last
// (their outputs are not stored).
static_assert(16 * (kDSlots - 2) + 15 < kDQuantDma, "slots before the last are quant slots");
struct DmaSlots {
  const uint8_t *base[kDSlots - 1];  // quant slots: the record half of chunk 0 (wave-uniform)
  const uint8_t *last;               // the last slot: this lane's 16 source bytes, chunk 0
  lds_void *dst[kDSlots];            // the slot's LDS destination, stage 0 (wave-uniform)
  int stage_bytes[kDSlots];          // LDS bytes from stage 0 to stage 1
  int blk[kDSlots];                  // block of the chunk the slot moves
  bool on_last;                      // this lane takes part in the last slot
};

__device__ __forceinline__ void dma_slots(DmaSlots &d, int8_t *qs, uint16_t *dsh,
                                          const uint8_t *tx, const uint8_t *ty, size_t gx0,
                                          size_t ngx, size_t gy0, size_t ngy, size_t nb,
                                          int wave, int lane) {
  auto record = [&](int g, int b) {
    return g < 4 ? tx + (min(gx0 + g, ngx - 1) * nb + b) * kTRec
                 : ty + (min(gy0 + (g - 4), ngy - 1) * nb + b) * kTRec;
  };
#pragma unroll
  for (int k = 0; k < kDSlots; ++k) {
    const int j = min(wave + 16 * k, kDDma - 1);  // slots past kDDma are never issued
    if (j < kDQuantDma) {
      const int b = j / 12, h = (j / 6) & 1, g = j % 6;
      if (k + 1 < kDSlots)
        d.base[k] = record(g, b) + h * 1024;
      else
        d.last = record(g, b) + h * 1024 + lane * 16;
      // a generic pointer into LDS -> the LDS address space (what the DMA takes)
      d.dst[k] = (lds_void *)(qs + b * kDBlock + h * kDHalf + g * kTG * 16);
      d.stage_bytes[k] = kDStage;
      d.blk[k] = b;
      if (k + 1 == kDSlots)
        d.on_last = true;
    } else {
      const int b = j - kDQuantDma;
      d.last = record(min(lane >> 3, 5), b) + 2048 + (lane & 7) * 16;
      d.dst[k] = (lds_void *)(dsh + b * kDHRow);
      d.stage_bytes[k] = kDKB * kDHRow * 2;
      d.blk[k] = b;
      d.on_last = lane < 48;
    }
  }
}

// Issues slot k of this wave's DMA of K chunk c (nbc blocks) into stage st;
// returns 1 if the slot moves a block of the chunk, else 0.  kBuf: the quant
// slots as buffer loads (buffer_load_dwordx4 ... offen lds: the slot's chunk-0
// record half as the resource base in scalar registers, the chunk offset as
// soffset, one 32-bit lane offset shared by every slot) instead of
// global_load_lds with a 64-bit vector address per slot; the chunk offset is
// then 32-bit (nb * kTRec < 2^32, which the entries check).  The Q8_0 kernel
// takes it (4096^3 tiles 171.1 -> 169.1 us, 110 instead of 118 VGPRs,
// interleaved A/B); the Q4_0 kernel, at its register limit, would spill 18-20
// SGPRs.
template <bool kBuf>
__device__ __forceinline__ int dma_slot(const DmaSlots &d, int k, size_t c, int nbc, int st,
                                        int wave, int lane) {
  if (wave + 16 * k >= kDDma || d.blk[k] >= nbc)
    return 0;
  const size_t coff = c * kDKB * kTRec;
  lds_void *to =
      (lds_void *)((char __attribute__((address_space(3))) *)d.dst[k] + st * d.stage_bytes[k]);
  if (k + 1 < kDSlots) {
    if constexpr (kBuf) {
      // no stride; every 32-bit offset in range (the addresses are the ones the
      // global form would use); dword 3: 32-bit data format, as buffer_load_dword*
      // takes it on gfx9
      const __amdgpu_buffer_rsrc_t r =
          __builtin_amdgcn_make_buffer_rsrc((void *)d.base[k], (short)0, -1, 0x00020000);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, to, 16, static_cast<unsigned>(lane * 16),
                                               static_cast<unsigned>(coff), 0, 0);
    } else {
      __builtin_amdgcn_global_load_lds(d.base[k] + coff + lane * 16, to, 16, 0, 0);
    }
  } else if (d.on_last) {
    __builtin_amdgcn_global_load_lds(d.last + coff, to, 16, 0, 0);
  }
  return 1;
}

// Issues this wave's whole DMA of K chunk c into stage st (the prologue);
// returns how many DMA instructions it issued.
template <bool kBuf>
__device__ __forceinline__ int dma_chunk(const DmaSlots &d, size_t c, int nbc, int st,
                                         int wave, int lane) {
  int issued = 0;
#pragma unroll
  for (int k = 0; k < kDSlots; ++k)
    issued += dma_slot<kBuf>(d, k, c, nbc, st, wave, lane);
  return issued;
}

// Where a wave issues its DMA of the next chunk.  A global_load_lds leaves
// the wave only once the CU takes it -- about one instruction per 14 cycles
// per CU, one per ~68 cycles from a lone wave -- and costs its SIMD ~24-36
// MFMA-pipe cycles even then (probe kernels mixing MFMA chains with LDS DMA).
// All 16 waves issuing their ~5 slots right after the barrier queue together
// and the four waves of a SIMD stall at once: ~700 cycles of a ~7700-cycle
// chunk (per-wave cycle counters, Q8_0 4096^3).  kDmaSpread: slot k is issued
// after fold step k instead, between the wave's MFMAs (Q8_0 4096^3 tiles
// 0.2-2 % faster on four boxes, interleaved A/B).  The Q4_0 kernel keeps the
// DMA at the chunk's start: it is at its register limit, and every spread
// placement spills.
template <bool kQ4>
constexpr bool kDmaSpread = !kQ4;
static_assert(kDSlots <= 2 * kDKB, "a spread chunk issues one slot per fold step");

// Waits until at most `pending` of this wave's memory loads are outstanding
// (the DMA of the newest chunk; every older chunk has landed in LDS) and all
// its LDS reads are done, then meets the other waves at a barrier: after it,
// every wave's DMA of the older chunks is visible and no wave still reads the
// stage the next DMA overwrites.  s_waitcnt takes an immediate, hence the
// switch (gfx9 encoding: vmcnt in bits 3:0, expcnt 6:4 = 7 (no wait), lgkmcnt
// 11:8 = 0).  `before_barrier` runs between the wait and the barrier (what it
// writes to LDS is complete before the barrier: its lgkmcnt is waited too).
template <typename BeforeBarrier>
__device__ __forceinline__ void wait_dma_barrier(int pending, BeforeBarrier &&before_barrier) {
  switch (__builtin_amdgcn_readfirstlane(pending)) {  // the same in every lane
  case 0: __builtin_amdgcn_s_waitcnt(0x070); break;
  case 1: __builtin_amdgcn_s_waitcnt(0x071); break;
  case 2: __builtin_amdgcn_s_waitcnt(0x072); break;
  case 3: __builtin_amdgcn_s_waitcnt(0x073); break;
  case 4: __builtin_amdgcn_s_waitcnt(0x074); break;
  case 5: __builtin_amdgcn_s_waitcnt(0x075); break;
  case 6: __builtin_amdgcn_s_waitcnt(0x076); break;
  default: __builtin_amdgcn_s_waitcnt(0x077); break;
  }
  before_barrier();
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): its LDS writes are done
  __builtin_amdgcn_s_barrier();
}

__device__ __forceinline__ void wait_dma_barrier(int pending) {
  wait_dma_barrier(pending, [] {});
}

// The Q4_0 fold reads d_y as fp32 (mfma_fold.h, q4_fold).  The wave whose DMA
// slot brings block b's scales (slot kDQuantDma + b of the chunk, wave
// (kDQuantDma + b) % 16) widens that block's kDBN token scales once its own
// loads have landed -- the vmcnt wait alone orders them for the wave itself --
// into the fp32 row `fy` of the chunk's stage, before the barrier that
// publishes the chunk; two scales per lane.  dsh_st: the stage's fp16 scales.
__device__ __forceinline__ void widen_token_scales(const uint16_t *dsh_st, float *fy_st,
                                                   int nbc, int wave, int lane) {
#pragma unroll
  for (int b = 0; b < kDKB; ++b) {
    if ((kDQuantDma + b) % 16 == wave && b < nbc) {
#pragma unroll
      for (int k = 0; k < kDBN / 64; ++k) {
        const int t = lane + 64 * k;
        fy_st[b * kDBN + t] =
            static_cast<float>(__builtin_bit_cast(_Float16, dsh_st[b * kDHRow + kDBM + t]));
      }
    }
  }
}

// Work-group: 256 weight rows x 128 tokens, 16 waves, each wave two 32x32
// tiles stacked in M (64 weight rows x 32 tokens); K chunks of kDKB blocks in
// kDStages LDS stages: the DMA of the next kDStages-1 chunks is in flight while
// chunk c is folded, and the barrier after chunk c waits for chunk c+1's.
// kQ4: the weight tiles (tx) hold Q4_0 rows decoded to int8 (nibble - 8) and
// the fold is the Q4_0 one, fma(fl((float)sumi * d_x), d_y, acc), on
// transposed 32x32 tiles (tokens x weights; fold_chunk_q4); otherwise both
// sides are Q8_0 and the fold is fma((float)sumi, d_x * d_y, acc).
template <bool kPipe, bool kQ4>
__device__ __forceinline__ void gemm_tiles_body(size_t nb, float *s, const uint8_t *tx,
                                                const uint8_t *ty, size_t nr, size_t nc,
                                                size_t bs, int8_t *qs, uint16_t *dsh, float *fyd) {

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave >> 2, wn = wave & 3;  // 64 weight rows x 32 tokens per wave
  const int li = lane & 31, h = lane >> 5;
  const unsigned tiles_m = static_cast<unsigned>((nr + kDBM - 1) / kDBM);
  const unsigned tiles_n = static_cast<unsigned>((nc + kDBN - 1) / kDBN);
  unsigned tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const size_t m0 = static_cast<size_t>(tm) * kDBM;
  const size_t n0 = static_cast<size_t>(tn) * kDBN;
  const size_t ngx = (nr + kTG - 1) / kTG, ngy = (nc + kTG - 1) / kTG;
  const size_t gx0 = m0 / kTG, gy0 = n0 / kTG;

  float acc[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      acc[i][e] = 0.0f;

  if (tid < kDStages * kDKB * 32)  // the zero rows of every stage
    dsh[(tid >> 5) * kDHRow + kDRows + (tid & 31)] = 0;
  const size_t nchunks = (nb + kDKB - 1) / kDKB;
  const size_t nfull = nb / kDKB;
  auto blocks_of = [&](size_t c) {
    return static_cast<int>(min(static_cast<size_t>(kDKB), nb - c * kDKB));
  };
  DmaSlots slots;
  dma_slots(slots, qs, dsh, tx, ty, gx0, ngx, gy0, ngy, nb, wave, lane);
  constexpr int kAhead = kDStages - 1;  // chunks in flight beyond the one folded
  constexpr int kHStage = kDKB * kDHRow;
  constexpr int kFyStage = kDKB * kDBN;
  // what runs between a chunk's DMA wait and the barrier that publishes it:
  // the Q4_0 fold's fp32 token scales of chunk cc (in stage sc)
  auto publish = [&](size_t cc, int sc) {
    if constexpr (kQ4) {
      if (cc < nchunks)
        widen_token_scales(dsh + sc * kHStage, fyd + sc * kFyStage, blocks_of(cc), wave, lane);
    }
  };
  dma_chunk<!kQ4>(slots, 0, blocks_of(0), 0, wave, lane);
  int pending =
      kAhead > 1 && nchunks > 1 ? dma_chunk<!kQ4>(slots, 1, blocks_of(1), 1, wave, lane) : 0;
  // chunk 0 is in LDS, the zero rows written
  wait_dma_barrier(pending, [&] { publish(0, 0); });

  // this lane's operands in stage 0, block 0, for the wave's first tile
  const int8_t *qa0 = qs + (h * kDRows + wm * 64 + li) * 16;
  const int8_t *qb0 = qs + (h * kDRows + kDBM + wn * 32 + li) * 16;
  const uint16_t *hx0 = dsh + (h ? kDRows + li : wm * 64 + li);
  const uint16_t *hx1 = dsh + (h ? kDRows + li : wm * 64 + 32 + li);
  const uint16_t *hy = dsh + (h ? kDRows + li : kDBM + wn * 32 + li);

  // the Q4_0 fold (transposed tiles): d_x of the lane's weight row of tile 0,
  // the fp32 d_y of its tokens 4h.. (4 of every 8)
  const uint16_t *qx = dsh + wm * 64 + li;
  const float *qy = fyd + wn * 32 + 4 * h;

  int st = 0;  // stage of chunk c
  size_t c = 0;
  // One full chunk: the DMA of chunk c + kAhead is issued (before the fold or
  // between its steps), chunk c folded, and the barrier passed once chunk c + 1
  // is in LDS (with one chunk ahead it is the newest DMA).
  auto chunk = [&](auto fold) {
    const int sta = st + kAhead >= kDStages ? st + kAhead - kDStages : st + kAhead;
    const bool ahead = c + kAhead < nchunks;
    const int nba = ahead ? blocks_of(c + kAhead) : 0;
    if constexpr (kDmaSpread<kQ4>) {
      pending = 0;
      fold([&](int s) {
        if (s < kDSlots && ahead)
          pending += dma_slot<!kQ4>(slots, s, c + kAhead, nba, sta, wave, lane);
      });
    } else {
      pending = ahead ? dma_chunk<!kQ4>(slots, c + kAhead, nba, sta, wave, lane) : 0;
      fold([](int) {});
    }
    const int stn = st + 1 == kDStages ? 0 : st + 1;
    wait_dma_barrier(kAhead > 1 ? pending : 0, [&] { publish(c + 1, stn); });
    st = stn;
  };
  const int nbc = static_cast<int>(nb - nfull * kDKB);
  if constexpr (kQ4) {
    // the fast fold until a chunk holds a non-finite d_x among the wave's rows,
    // the exact one from there on (and for the partial tail, always)
    for (; c < nfull; ++c) {
      if (q4_chunk_nonfinite<kDHRow>(dsh + st * kHStage + wm * 64, kDKB, lane))
        break;
      chunk([&](auto after_step) {
        fold_chunk_q4<false, kDKB, kDBlock, 32 * 16, kDHRow, kDBN>(
            acc, qa0 + st * kDStage, qb0 + st * kDStage, qx + st * kHStage, qy + st * kFyStage,
            after_step);
      });
    }
    for (; c < nfull; ++c)
      chunk([&](auto after_step) {
        fold_chunk_q4<true, kDKB, kDBlock, 32 * 16, kDHRow, kDBN>(
            acc, qa0 + st * kDStage, qb0 + st * kDStage, qx + st * kHStage, qy + st * kFyStage,
            after_step);
      });
    if (nbc > 0)
      fold_tail_q4<true, kDBlock, 32 * 16, kDHRow, kDBN>(acc, qa0 + st * kDStage,
                                                         qb0 + st * kDStage, qx + st * kHStage,
                                                         qy + st * kFyStage, nbc);
  } else {
    for (; c < nfull; ++c)
      chunk([&](auto after_step) {
        fold_chunk_q8<kPipe, kDKB, kDBlock, 32 * 16, kDHRow>(
            acc, qa0 + st * kDStage, qb0 + st * kDStage, hx0 + st * kHStage,
            hx1 + st * kHStage, hy + st * kHStage, after_step);
      });
    if (nbc > 0)
      fold_tail_q8<kDBlock, 32 * 16, kDHRow>(acc, qa0 + st * kDStage, qb0 + st * kDStage,
                                             hx0 + st * kHStage, hx1 + st * kHStage,
                                             hy + st * kHStage, nbc);
  }

  if constexpr (kQ4) {
    // Lane (li, h) holds weight row li of each tile and tokens 8g + 4h + j:
    // stored directly, every store would scatter over 32 rows.  Each tile goes
    // through a wave-private 32x32 fp32 buffer in LDS instead (row-major,
    // padded to 33 floats a row: no bank conflicts either way), read back as
    // 32 consecutive tokens of one row per half-wave.  The buffers lie in the
    // quant stage the last full chunk used: no wave reads it after that
    // chunk's barrier (the tail, if any, reads the other stage) and no DMA
    // targets it.
    float *tb = reinterpret_cast<float *>(qs + (nbc > 0 ? 1 - st : st) * kDStage) + wave * 32 * 33;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        tb[li * 33 + 8 * (e >> 2) + 4 * h + (e & 3)] = acc[i][e];
      __builtin_amdgcn_wave_barrier();
      const size_t col = n0 + wn * 32 + li;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int r = 2 * k + h;  // this half-wave's weight row of the tile
        const size_t row = m0 + wm * 64 + i * 32 + r;
        const float v = tb[r * 33 + li];
        if (row < nr && col < nc)
          s[row * bs + col] = v;
      }
      __builtin_amdgcn_wave_barrier();
    }
  } else {
    const size_t col = n0 + wn * 32 + li;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const size_t row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < nr && col < nc)
          s[row * bs + col] = acc[i][e];
      }
  }
}

template <bool kPipe>
__global__ __launch_bounds__(kDThreads, 1) void gemm_tiles_q8(size_t nb, float *s,
                                                              const uint8_t *tx,
                                                              const uint8_t *ty, size_t nr,
                                                              size_t nc, size_t bs) {
  __shared__ __align__(16) int8_t qs[kDStages * kDStage];
  __shared__ __align__(16) uint16_t dsh[kDStages * kDKB * kDHRow];
  gemm_tiles_body<kPipe, false>(nb, s, tx, ty, nr, nc, bs, qs, dsh, nullptr);
}

__global__ __launch_bounds__(kDThreads, 1) void gemm_tiles_q4(size_t nb, float *s,
                                                              const uint8_t *tx,
                                                              const uint8_t *ty, size_t nr,
                                                              size_t nc, size_t bs) {
  __shared__ __align__(16) int8_t qs[kDStages * kDStage];
  __shared__ __align__(16) uint16_t dsh[kDStages * kDKB * kDHRow];
  __shared__ __align__(16) float fyd[kDStages * kDKB * kDBN];
  gemm_tiles_body<true, true>(nb, s, tx, ty, nr, nc, bs, qs, dsh, fyd);
}

// ---- the Q8_0 GEMM on 256 x 256 work-group tiles ----------------------------
// 8 waves, two per SIMD, each folding 64 weight rows x 128 tokens (2 x 4 tiles,
// 128 accumulator registers of the 256 a wave may hold at two waves per SIMD).
// Against the 256 x 128 tile a K block's 512 staged rows feed twice the tiles:
// a third fewer DMA instructions and half the LDS operand reads per tile and
// block, and a 4096 x 4096 output is 256 work-groups, one per CU.  K chunks of
// kEKB blocks in two LDS stages.  Wave w's DMA is its own row group's records
// (groups 0-3 the weight tile's, 4-7 the token tile's): both halves of each of
// the chunk's blocks, 1 KB per instruction from one scalar base; waves 0-3
// also move the scales of block w (64 lanes: group l / 8, 16 bytes l % 8).
constexpr int kEBM = 256, kEBN = 256, kEKB = 4;
constexpr int kERows = kEBM + kEBN;   // 512 staged rows
constexpr int kEHalf = kERows * 16;   // 8192: one half of one block, all rows
constexpr int kEBlock = 2 * kEHalf;   // 16384
constexpr int kEStage = kEKB * kEBlock;
// fp16 scales per block row: 512 rows, then 128 zero rows (lanes 32-63 of
// every tile, at its tile offset of up to 96 rows, read zeros: k-slots 4-7 of
// the scale MFMA)
constexpr int kEHRow = kERows + 128;
constexpr int kEThreads = 512;
constexpr int kEStages = 2;
constexpr int kEQuantSlots = 2 * kEKB;  // quant DMA instructions per wave and chunk
static_assert(kEStages * (kEStage + kEKB * kEHRow * 2) <= 160 * 1024,
              "the stages fit the 160 KB of LDS");
static_assert(kEKB <= 4, "the scale moves of a chunk are waves 0-3's");

// kQ4: the weight groups hold Q4_0 rows decoded to int8 (as gemm_tiles_q4's)
// and the fold is the Q4_0 one on transposed tiles (fold_chunk_q4_2x4): the
// waves that move a block's scales (waves 0-3, block w) also widen its 256
// token scales to the fp32 row fyd before the barrier that publishes the
// chunk, the fast fold runs until a chunk holds a non-finite d_x among the
// wave's weight rows, and each tile is stored through a wave-private LDS
// buffer (as gemm_tiles_body's Q4_0 stores).
constexpr int kEFyStage = kEKB * kEBN;  // fp32 token scales per stage
static_assert(kEStages * (kEStage + kEKB * kEHRow * 2 + kEFyStage * 4) <= 160 * 1024,
              "the Q4_0 stages fit the 160 KB of LDS");

// LDS DMA written as inline assembly, for code whose DMA the compiler must not
// track (the exact-form loop of the 256 x 256 Q4_0 kernel).  The compiler then
// inserts no wait for these loads: the kernels wait for them explicitly (the
// vmcnt wait before each chunk's barrier), as they do for the intrinsic form.
// M0 (the LDS destination) is saved and restored around the instruction, and
// "memory" keeps every other memory access on its side of it.
typedef unsigned v4u __attribute__((ext_vector_type(4)));

// buffer_load_dwordx4 ... offen lds: 16 bytes per lane from base + soff + voff
// (resource: no stride, every 32-bit offset in range, dword 3 as
// __builtin_amdgcn_make_buffer_rsrc takes it) into LDS at `to` + 16 * lane.
__device__ __forceinline__ void buffer_load_lds_asm(const uint8_t *base, unsigned voff,
                                                    unsigned soff, lds_void *to) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const v4u rsrc = {
      static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<unsigned>(a))),
      static_cast<unsigned>(
          __builtin_amdgcn_readfirstlane(static_cast<unsigned>(a >> 32) & 0xFFFFu)),
      0xFFFFFFFFu, 0x00020000u};
  const unsigned m0 = static_cast<unsigned>(
      __builtin_amdgcn_readfirstlane(static_cast<unsigned>(reinterpret_cast<uintptr_t>(to))));
  const unsigned so = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(soff));
  unsigned saved;
  asm volatile("s_mov_b32 %0, m0\n\t"
               "s_mov_b32 m0, %1\n\t"
               "s_nop 0\n\t"
               "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
               "s_mov_b32 m0, %0"
               : "=&s"(saved)
               : "s"(m0), "v"(voff), "s"(rsrc), "s"(so)
               : "memory");
}

// global_load_lds_dwordx4: 16 bytes per lane from `from` into LDS at `to` +
// 16 * lane.
__device__ __forceinline__ void global_load_lds_asm(const uint8_t *from, lds_void *to) {
  const unsigned m0 = static_cast<unsigned>(
      __builtin_amdgcn_readfirstlane(static_cast<unsigned>(reinterpret_cast<uintptr_t>(to))));
  unsigned saved;
  asm volatile("s_mov_b32 %0, m0\n\t"
               "s_mov_b32 m0, %1\n\t"
               "s_nop 0\n\t"
               "global_load_lds_dwordx4 %2, off\n\t"
               "s_mov_b32 m0, %0"
               : "=&s"(saved)
               : "s"(m0), "v"(from)
               : "memory");
}

// One wave's view of a 256 x 256 work-group: its tile, its DMA slots and the
// LDS operands of its lanes.
struct Tiles256 {
  int wave, lane, wm, wn, li, h;  // wm, wn: 64 weight rows x 128 tokens per wave
  size_t m0, n0, nb, nchunks;
  const uint8_t *own;  // the wave's row group's records (wave-uniform)
  const uint8_t *scl;  // this lane's 16 scale bytes of block `wave` of chunk 0
  int8_t *qs;
  uint16_t *dsh;
  float *fyd;

  __device__ Tiles256(size_t nb_, const uint8_t *tx, const uint8_t *ty, size_t nr, size_t nc,
                      int8_t *qs_, uint16_t *dsh_, float *fyd_)
      : nb(nb_), qs(qs_), dsh(dsh_), fyd(fyd_) {
    const int tid = threadIdx.x;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    lane = tid & 63;
    wm = wave & 3;
    wn = wave >> 2;
    li = lane & 31;
    h = lane >> 5;
    const unsigned tiles_m = static_cast<unsigned>((nr + kEBM - 1) / kEBM);
    const unsigned tiles_n = static_cast<unsigned>((nc + kEBN - 1) / kEBN);
    unsigned tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    m0 = static_cast<size_t>(tm) * kEBM;
    n0 = static_cast<size_t>(tn) * kEBN;
    const size_t ngx = (nr + kTG - 1) / kTG, ngy = (nc + kTG - 1) / kTG;
    const size_t gx0 = m0 / kTG, gy0 = n0 / kTG;
    // row group g's records (groups past an operand's last re-read the last;
    // their outputs are not stored)
    auto group = [&](int g) {
      return g < 4 ? tx + min(gx0 + g, ngx - 1) * nb * kTRec
                   : ty + min(gy0 + (g - 4), ngy - 1) * nb * kTRec;
    };
    own = group(wave);
    scl = group(lane >> 3) + static_cast<size_t>(wave) * kTRec + 2048 + (lane & 7) * 16;
    nchunks = (nb + kEKB - 1) / kEKB;
  }

  __device__ int blocks_of(size_t c) const {
    return static_cast<int>(min(static_cast<size_t>(kEKB), nb - c * kEKB));
  }

  // Slot k < kEQuantSlots of chunk c into stage st: half k & 1 of block k >> 1
  // (buffer form: the wave's records as the resource base in scalar registers,
  // the chunk's offset in them as soffset, 32-bit as the entries check); slot
  // kEQuantSlots: the scales of block `wave`.  Returns 1 if it moved anything.
  // kAsm: the same two instructions as inline assembly (buffer_load_lds_asm,
  // global_load_lds_asm), which the compiler does not see as LDS writes.
  template <bool kAsm = false>
  __device__ int slot(int k, size_t c, int nbc, int st) const {
    if (k < kEQuantSlots) {
      if ((k >> 1) >= nbc)
        return 0;
      lds_void *to = (lds_void *)(qs + st * kEStage + (k >> 1) * kEBlock + (k & 1) * kEHalf +
                                  wave * kTG * 16);
      const unsigned off = static_cast<unsigned>((c * kEKB + (k >> 1)) * kTRec + (k & 1) * 1024);
      if constexpr (kAsm) {
        buffer_load_lds_asm(own, static_cast<unsigned>(lane * 16), off, to);
      } else {
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc((void *)own, (short)0, -1, 0x00020000);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, to, 16, static_cast<unsigned>(lane * 16),
                                                 off, 0, 0);
      }
      return 1;
    }
    if (wave >= nbc)
      return 0;
    const uint8_t *from = scl + c * kEKB * kTRec;
    lds_void *to = (lds_void *)(dsh + st * kEKB * kEHRow + wave * kEHRow);
    if constexpr (kAsm)
      global_load_lds_asm(from, to);
    else
      __builtin_amdgcn_global_load_lds(from, to, 16, 0, 0);
    return 1;
  }

  // Between a chunk's DMA wait and its barrier: the Q4_0 fold's fp32 token
  // scales of chunk cc in stage sc, widened by the wave that moved them (its
  // own loads have landed after its wait), four per lane.
  __device__ void publish_q4(size_t cc, int sc) const {
    if (cc < nchunks && wave < blocks_of(cc)) {
#pragma unroll
      for (int k = 0; k < kEBN / 64; ++k) {
        const int t = lane + 64 * k;
        fyd[sc * kEFyStage + wave * kEBN + t] = static_cast<float>(__builtin_bit_cast(
            _Float16, dsh[sc * kEKB * kEHRow + wave * kEHRow + kEBM + t]));
      }
    }
  }

  // this lane's operands in stage 0, block 0, tile 0 (lanes 32-63: half 1 of the
  // quants; for the Q8_0 fold the zero scale rows)
  __device__ const int8_t *qa() const { return qs + (h * kERows + wm * 64 + li) * 16; }
  __device__ const int8_t *qb() const { return qs + (h * kERows + kEBM + wn * 128 + li) * 16; }
  __device__ const uint16_t *hx() const { return dsh + (h ? kERows + li : wm * 64 + li); }
  __device__ const uint16_t *hy() const { return dsh + (h ? kERows + li : kEBM + wn * 128 + li); }
  // the Q4_0 fold: d_x of the lane's weight row li, fp32 d_y of its tokens 4h..
  __device__ const uint16_t *q4x() const { return dsh + wm * 64 + li; }
  __device__ const float *q4y() const { return fyd + wn * 128 + 4 * h; }
};

// Full chunk c of the 256 x 256 kernel in stage st: the fold (`fold(after_step)`,
// slot k of chunk c + 1 issued after its step 3k), then the wait for chunk c + 1,
// `publish(c + 1, stage)` and the barrier.  Returns the stage of chunk c + 1.
template <bool kAsm = false, typename Fold, typename Publish>
__device__ __forceinline__ int chunk256(const Tiles256 &t, size_t c, int st, Fold &&fold,
                                        Publish &&publish) {
  const bool ahead = c + 1 < t.nchunks;
  const int nba = ahead ? t.blocks_of(c + 1) : 0;
  const int sta = st ^ 1;
  fold([&](int s) {
    if (s % 3 == 0 && s / 3 <= kEQuantSlots && ahead)
      t.template slot<kAsm>(s / 3, c + 1, nba, sta);
  });
  wait_dma_barrier(0, [&] { publish(c + 1, sta); });  // no wave reads stage st any more
  return sta;
}

template <bool kQ4>
__device__ __forceinline__ void gemm_tiles256_body(size_t nb, float *s, const uint8_t *tx,
                                                   const uint8_t *ty, size_t nr, size_t nc,
                                                   size_t bs, int8_t *qs, uint16_t *dsh,
                                                   float *fyd) {
  const Tiles256 t(nb, tx, ty, nr, nc, qs, dsh, fyd);
  const int tid = threadIdx.x, li = t.li, h = t.h, wm = t.wm, wn = t.wn;
  constexpr int kHStage = kEKB * kEHRow;

  float acc[2][4][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc[i][j][e] = 0.0f;

  if constexpr (!kQ4)
    for (int k = tid; k < kEStages * kEKB * 128; k += kEThreads)  // the zero rows
      dsh[(k >> 7) * kEHRow + kERows + (k & 127)] = 0;

  auto publish = [&](size_t cc, int sc) {
    if constexpr (kQ4)
      t.publish_q4(cc, sc);
  };
#pragma unroll
  for (int k = 0; k <= kEQuantSlots; ++k)
    t.slot(k, 0, t.blocks_of(0), 0);
  wait_dma_barrier(0, [&] { publish(0, 0); });  // chunk 0 is in LDS, the zero rows written

  const int8_t *qa = t.qa(), *qb = t.qb();
  int st = 0;
  size_t c = 0;
  const size_t nfull = nb / kEKB;
  const int nbc = static_cast<int>(nb - nfull * kEKB);
  const size_t m0 = t.m0, n0 = t.n0;
  if constexpr (kQ4) {
    const uint16_t *qx = t.q4x();
    const float *qy = t.q4y();
    // The fast fold until a chunk holds a non-finite d_x among the wave's
    // weight rows, then the exact one.  The exact loop issues its DMA as
    // inline assembly: with a second copy of the DMA intrinsics in the kernel,
    // the compiler makes every LDS read of the fast loop that follows a DMA
    // issue wait for that DMA (4096^3 185 against 155 us).
    for (; c < nfull; ++c) {
      if (q4_chunk_nonfinite<kEHRow>(dsh + st * kHStage + wm * 64, kEKB, t.lane))
        break;
      st = chunk256(
          t, c, st,
          [&](auto after_step) {
            fold_chunk_q4_2x4<false, kEKB, kEBlock, 32 * 16, kEHRow, kEBN>(
                acc, qa + st * kEStage, qb + st * kEStage, qx + st * kHStage,
                qy + st * kEFyStage, after_step);
          },
          publish);
    }
    for (; c < nfull; ++c)
      st = chunk256<true>(
          t, c, st,
          [&](auto after_step) {
            fold_chunk_q4_2x4<true, kEKB, kEBlock, 32 * 16, kEHRow, kEBN>(
                acc, qa + st * kEStage, qb + st * kEStage, qx + st * kHStage,
                qy + st * kEFyStage, after_step);
          },
          publish);
    if (nbc > 0)
      fold_tail_q4_2x4<true, kEBlock, 32 * 16, kEHRow, kEBN>(
          acc, qa + st * kEStage, qb + st * kEStage, qx + st * kHStage, qy + st * kEFyStage, nbc);
    // Lane (li, h) holds weight row li of tile (i, j) and its tokens 8g + 4h + e:
    // each tile goes through a wave-private 32 x 33 fp32 buffer in the quant
    // stage no wave reads any more (the last full chunk's if a tail follows,
    // else the other) and is stored as 32 consecutive tokens of one row per
    // half-wave.
    float *tb =
        reinterpret_cast<float *>(qs + (nbc > 0 ? 1 - st : st) * kEStage) + t.wave * 32 * 33;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int e = 0; e < 16; ++e)
          tb[li * 33 + 8 * (e >> 2) + 4 * h + (e & 3)] = acc[i][j][e];
        __builtin_amdgcn_wave_barrier();
        const size_t col = n0 + wn * 128 + j * 32 + li;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const int r = 2 * k + h;  // this half-wave's weight row of the tile
          const size_t row = m0 + wm * 64 + i * 32 + r;
          const float v = tb[r * 33 + li];
          if (row < nr && col < nc)
            s[row * bs + col] = v;
        }
        __builtin_amdgcn_wave_barrier();
      }
  } else {
    const uint16_t *hx = t.hx(), *hy = t.hy();
    for (; c < nfull; ++c)
      st = chunk256(
          t, c, st,
          [&](auto after_step) {
            fold_chunk_q8_2x4<kEKB, kEBlock, 32 * 16, kEHRow>(
                acc, qa + st * kEStage, qb + st * kEStage, hx + st * kHStage, hy + st * kHStage,
                after_step);
          },
          publish);
    if (nbc > 0)
      fold_tail_q8_2x4<kEBlock, 32 * 16, kEHRow>(acc, qa + st * kEStage, qb + st * kEStage,
                                                 hx + st * kHStage, hy + st * kHStage, nbc);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const size_t col = n0 + wn * 128 + j * 32 + li;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const size_t row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
          if (row < nr && col < nc)
            s[row * bs + col] = acc[i][j][e];
        }
    }
  }
}

__global__ __launch_bounds__(kEThreads, 1) void gemm_tiles256_q8(size_t nb, float *s,
                                                                 const uint8_t *tx,
                                                                 const uint8_t *ty, size_t nr,
                                                                 size_t nc, size_t bs) {
  __shared__ __align__(16) int8_t qs[kEStages * kEStage];
  __shared__ __align__(16) uint16_t dsh[kEStages * kEKB * kEHRow];
  gemm_tiles256_body<false>(nb, s, tx, ty, nr, nc, bs, qs, dsh, nullptr);
}

__global__ __launch_bounds__(kEThreads, 1) void gemm_tiles256_q4(size_t nb, float *s,
                                                                 const uint8_t *tx,
                                                                 const uint8_t *ty, size_t nr,
                                                                 size_t nc, size_t bs) {
  __shared__ __align__(16) int8_t qs[kEStages * kEStage];
  __shared__ __align__(16) uint16_t dsh[kEStages * kEKB * kEHRow];
  __shared__ __align__(16) float fyd[kEStages * kEFyStage];
  gemm_tiles256_body<true>(nb, s, tx, ty, nr, nc, bs, qs, dsh, fyd);
}

// ---- few work-group tiles: one 32 x 32 tile a wave, no LDS -----------------
// Where the 256-row tiles leave most CUs idle (a few hundred tokens against a
// few thousand weight rows: 4096 x 128 is 16 work-groups of 256 x 128), each
// wave folds one 32 x 32 output tile and a work-group of 4 waves covers one
// 64-row record group of each operand (64 weight rows x 64 tokens).  A record
// half is exactly a v_mfma_i32_32x32x32_i8 operand of 32 rows (lane l: row
// l % 32, quants 16 (l / 32) .. + 15), so every operand is one 16-byte load per
// lane straight into registers, kSAhead blocks in flight, and the MFMAs of
// block b + 1 are issued before block b is folded.
//   Q8_0: acc = fma((float)sumi, d_x * d_y, acc), d_x * d_y from the f16 MFMA
//         (scales in k-slot 0 of lanes 0-31, zero elsewhere: exact products);
//   Q4_0: acc = fma(fl((float)sumi * d_x), d_y, acc), the weight rows' d_x
//         spread over the tile by the same f16 MFMA against 1.0 (exact), the
//         lane's token scale d_y widened once per block.
// Rows and tokens past nr / nc are the zero rows of the last record group and
// are not stored.  Every output keeps its ascending-block fold: the same bits
// as the other tiled kernels.
constexpr int kSBM = 64, kSBN = 64;  // work-group tile (one record group each)
constexpr int kSAhead = 7;           // blocks in flight a wave (8: 12 bytes of spills)

struct Ops32 {
  v4i a, b;
  uint32_t ux, uy;
};

// One block of a wave's 32 x 32 tile: the block sums, the scale products (Q8_0)
// or the weight rows' d_x spread over the tile (Q4_0), and the lane's token
// scale (Q4_0).  kmask keeps the scale in k-slot 0 of lanes 0-31 only; one is
// fp16 1.0 there and 0 elsewhere.
struct Step32 {
  v16i sumi;
  v16f scl;
  float dy;
};

template <bool kQ4>
__device__ __forceinline__ Step32 issue32(const Ops32 &o, uint32_t kmask, uint32_t one) {
  Step32 t;
  t.sumi = q8_sumi(o.a, o.b);
  if constexpr (kQ4) {
    t.scl = q8_dxy(o.ux & kmask, one);
    t.dy = fp16_bits_to_f32(o.uy);
    asm volatile("" : "+v"(t.dy));  // widened once (not an fma_mix per output)
  } else {
    t.scl = q8_dxy(o.ux & kmask, o.uy & kmask);
    t.dy = 0.0f;
  }
  return t;
}

template <bool kQ4>
__device__ __forceinline__ void fold32(float (&acc)[16], const Step32 &t) {
  if constexpr (kQ4) {
#pragma unroll
    for (int e = 0; e < 16; ++e)
      acc[e] = fmaf(static_cast<float>(t.sumi[e]) * t.scl[e], t.dy, acc[e]);
  } else {  // all 16 conversions before the fmas, as q8_fold<true> (without its pin)
    float f[16];
#pragma unroll
    for (int e = 0; e < 16; ++e)
      f[e] = static_cast<float>(t.sumi[e]);
#pragma unroll
    for (int e = 0; e < 16; ++e)
      acc[e] = fmaf(f[e], t.scl[e], acc[e]);
  }
#pragma unroll
  for (int e = 0; e < 16; ++e)
    asm volatile("" : "+v"(acc[e]));
}

// Lane (li, h) of a 32 x 32 tile at weight row row0, token column col holds
// rows row0 + 8 (e / 4) + 4h + e % 4.
__device__ __forceinline__ void store32(float *s, const float (&acc)[16], size_t row0, size_t col,
                                        int h, size_t nr, size_t nc, size_t bs) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const size_t row = row0 + 8 * (e >> 2) + 4 * h + (e & 3);
    if (row < nr && col < nc)
      s[row * bs + col] = acc[e];
  }
}

// At most two waves a SIMD: every register is then a VGPR (a higher occupancy
// target puts the MFMA results in AGPRs, and each block then pays their copies
// out).  Two waves per tile, each folding half of the outputs after issuing
// the same loads and MFMAs, measured slower (4096 x 128 x 4096: 24.4 against
// 17.3 us).
template <bool kQ4>
__global__ __launch_bounds__(256, 2) void gemm_tiles32(unsigned nb, float *s, const uint8_t *tx,
                                                       const uint8_t *ty, size_t nr, size_t nc,
                                                       size_t bs) {
  const int lane = threadIdx.x & 63;
  const int tile = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int wm = tile & 1, wn = tile >> 1;  // the tile's 32-row halves of the two groups
  const int li = lane & 31, h = lane >> 5;
  const unsigned tiles_m = static_cast<unsigned>((nr + kSBM - 1) / kSBM);
  const unsigned tiles_n = static_cast<unsigned>((nc + kSBN - 1) / kSBN);
  unsigned tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const uint8_t *ra = tx + static_cast<size_t>(tm) * nb * kTRec;
  const uint8_t *rb = ty + static_cast<size_t>(tn) * nb * kTRec;
  // lane offsets within a record; the record base is wave-uniform (SGPRs)
  const unsigned qa = h * 1024 + (32 * wm + li) * 16, qb = h * 1024 + (32 * wn + li) * 16;
  const unsigned sa = 2 * kTG * 16 + (32 * wm + li) * 2, sb = 2 * kTG * 16 + (32 * wn + li) * 2;
  const uint32_t kmask = h ? 0u : 0xffffu;  // k-slot 0 of lanes 0-31 only
  const uint32_t one = h ? 0u : 0x3c00u;    // fp16 1.0
  const unsigned last = nb - 1;

  // Buffer loads: the record's address is the descriptor's base (SGPRs, one
  // per block and operand), the lane's 32-bit offset the VGPR offset, so no
  // load pays a 64-bit VALU address add (global loads from a 64-bit per-lane
  // address paid four a block: 4096 x 128 x 4096 21.8 -> 17.3 us).  Every
  // offset stays inside the 2176-byte record the descriptor spans.
  auto load = [&](unsigned b, Ops32 &o) {
    const __amdgpu_buffer_rsrc_t pa = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(ra + static_cast<size_t>(b) * kTRec), (short)0, kTRec, 0x00020000);
    const __amdgpu_buffer_rsrc_t pb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(rb + static_cast<size_t>(b) * kTRec), (short)0, kTRec, 0x00020000);
    o.a = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(pa, qa, 0, 0));
    o.b = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(pb, qb, 0, 0));
    o.ux = __builtin_amdgcn_raw_buffer_load_b16(pa, sa, 0, 0);
    o.uy = __builtin_amdgcn_raw_buffer_load_b16(pb, sb, 0, 0);
  };
  const auto issue = [&](const Ops32 &o) { return issue32<kQ4>(o, kmask, one); };
  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e)
    acc[e] = 0.0f;
  const auto fold = [&](const Step32 &t) { fold32<kQ4>(acc, t); };

  Ops32 ring[kSAhead];
#pragma unroll
  for (int j = 0; j < kSAhead; ++j)
    load(min(static_cast<unsigned>(j), last), ring[j]);
  Step32 cur = issue(ring[0]);
  load(min(static_cast<unsigned>(kSAhead), last), ring[0]);
  // block b + 1 sits in slot (b + 1) % kSAhead: its MFMAs go out before block
  // b's fold, and the slot is refilled with block b + 1 + kSAhead (clamped to
  // the last block, whose extra copies are never folded).  Whole rounds of
  // kSAhead blocks first, with no branch between the loads and their use, so
  // the waits count exactly the loads still in flight.
  auto step = [&](unsigned b, int j) {
    const int kn = (j + 1) % kSAhead;
    const Step32 nxt = issue(ring[kn]);
    load(min(b + 1 + kSAhead, last), ring[kn]);
    fold(cur);
    cur = nxt;
  };
  unsigned b0 = 0;
  for (; b0 + kSAhead <= nb; b0 += kSAhead) {
#pragma unroll
    for (int j = 0; j < kSAhead; ++j)
      step(b0 + j, j);
  }
#pragma unroll
  for (int j = 0; j < kSAhead - 1; ++j)
    if (b0 + j < nb)
      step(b0 + j, j);
  store32(s, acc, static_cast<size_t>(tm) * kSBM + 32 * wm,
          static_cast<size_t>(tn) * kSBN + 32 * wn + li, h, nr, nc, bs);
}

// ---- fewer still: one 16 x 16 tile a wave ----------------------------------
// Where even the 32 x 32 tiles leave most SIMDs without a wave (4096 weight
// rows x 64 tokens: 256 waves for 1024 SIMDs, each at one wave a SIMD, where
// the fold issues at ~6 cycles an instruction), a wave folds one 16 x 16 tile
// and a work-group of 4 waves a 32 x 32 tile (half of a record group's rows).  A
// v_mfma_i32_16x16x32_i8 lane holds 8 quants, lane l: row l % 16, quants
// 8 (l / 16) .. + 7 -- 8 bytes of one record half, so again one load per lane
// and operand; the f16 MFMA (16x16x16) gives d_x * d_y (Q8_0) or spreads d_x
// (Q4_0) as in the 32 x 32 kernel, from k-slot 0 of lanes 0-15.  Each output
// keeps its ascending-block fold: the same bits.
constexpr int kTBM = 32, kTBN = 32;  // work-group tile
constexpr int kTAhead = 12;          // blocks in flight a wave

typedef float v4f __attribute__((ext_vector_type(4)));

struct Ops16 {
  long a, b;
  uint32_t ux, uy;
};

struct Step16 {
  v4i sumi;
  v4f scl;
  float dy;
};

__device__ __forceinline__ v4h kslot0_16(uint32_t bits) {
  const v2h z = {};
  return __builtin_shufflevector(__builtin_bit_cast(v2h, bits), z, 0, 1, 2, 3);
}

template <bool kQ4>
__device__ __forceinline__ Step16 issue16(const Ops16 &o, uint32_t kmask, uint32_t one) {
  Step16 t;
  t.sumi = __builtin_amdgcn_mfma_i32_16x16x32_i8(o.a, o.b, v4i{}, 0, 0, 0);
  if constexpr (kQ4) {
    t.scl = __builtin_amdgcn_mfma_f32_16x16x16f16(kslot0_16(o.ux & kmask), kslot0_16(one),
                                                 v4f{}, 0, 0, 0);
    t.dy = fp16_bits_to_f32(o.uy);
    asm volatile("" : "+v"(t.dy));
  } else {
    t.scl = __builtin_amdgcn_mfma_f32_16x16x16f16(kslot0_16(o.ux & kmask),
                                                 kslot0_16(o.uy & kmask), v4f{}, 0, 0, 0);
    t.dy = 0.0f;
  }
  return t;
}

template <bool kQ4>
__device__ __forceinline__ void fold16(float (&acc)[4], const Step16 &t) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (kQ4)
      acc[e] = fmaf(static_cast<float>(t.sumi[e]) * t.scl[e], t.dy, acc[e]);
    else
      acc[e] = fmaf(static_cast<float>(t.sumi[e]), t.scl[e], acc[e]);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
    asm volatile("" : "+v"(acc[e]));
}

template <bool kQ4>
__global__ __launch_bounds__(256, 2) void gemm_tiles16(unsigned nb, float *s, const uint8_t *tx,
                                                    const uint8_t *ty, size_t nr, size_t nc,
                                                    size_t bs) {
  const int lane = threadIdx.x & 63;
  const int tile = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int wm = tile & 1, wn = tile >> 1;  // the wave's 16-row halves of the 32 x 32 tile
  const int li = lane & 15, q = lane >> 4;  // MFMA row / token li, quant group q
  const unsigned tiles_m = static_cast<unsigned>((nr + kTBM - 1) / kTBM);
  const unsigned tiles_n = static_cast<unsigned>((nc + kTBN - 1) / kTBN);
  unsigned tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  // weight rows 32 tm + 16 wm + li: record group tm / 2, row (tm % 2) * 32 + 16 wm + li
  const uint8_t *ra = tx + static_cast<size_t>(tm >> 1) * nb * kTRec;
  const uint8_t *rb = ty + static_cast<size_t>(tn >> 1) * nb * kTRec;
  const unsigned xr = (tm & 1) * 32 + 16 * wm + li, yr = (tn & 1) * 32 + 16 * wn + li;
  const unsigned qa = (q >> 1) * 1024 + xr * 16 + 8 * (q & 1);
  const unsigned qb = (q >> 1) * 1024 + yr * 16 + 8 * (q & 1);
  const unsigned sa = 2 * kTG * 16 + xr * 2, sb = 2 * kTG * 16 + yr * 2;
  const uint32_t kmask = q ? 0u : 0xffffu;  // k-slot 0 lives in lanes 0-15
  const uint32_t one = q ? 0u : 0x3c00u;
  const unsigned last = nb - 1;

  auto load = [&](unsigned b, Ops16 &o) {
    const __amdgpu_buffer_rsrc_t pa = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(ra + static_cast<size_t>(b) * kTRec), (short)0, kTRec, 0x00020000);
    const __amdgpu_buffer_rsrc_t pb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(rb + static_cast<size_t>(b) * kTRec), (short)0, kTRec, 0x00020000);
    o.a = __builtin_bit_cast(long, __builtin_amdgcn_raw_buffer_load_b64(pa, qa, 0, 0));
    o.b = __builtin_bit_cast(long, __builtin_amdgcn_raw_buffer_load_b64(pb, qb, 0, 0));
    o.ux = __builtin_amdgcn_raw_buffer_load_b16(pa, sa, 0, 0);
    o.uy = __builtin_amdgcn_raw_buffer_load_b16(pb, sb, 0, 0);
  };
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  Ops16 ring[kTAhead];
#pragma unroll
  for (int j = 0; j < kTAhead; ++j)
    load(min(static_cast<unsigned>(j), last), ring[j]);
  Step16 cur = issue16<kQ4>(ring[0], kmask, one);
  load(min(static_cast<unsigned>(kTAhead), last), ring[0]);
  auto step = [&](unsigned b, int j) {
    const int kn = (j + 1) % kTAhead;
    const Step16 nxt = issue16<kQ4>(ring[kn], kmask, one);
    load(min(b + 1 + kTAhead, last), ring[kn]);
    fold16<kQ4>(acc, cur);
    cur = nxt;
  };
  unsigned b0 = 0;
  for (; b0 + kTAhead <= nb; b0 += kTAhead) {
#pragma unroll
    for (int j = 0; j < kTAhead; ++j)
      step(b0 + j, j);
  }
#pragma unroll
  for (int j = 0; j < kTAhead - 1; ++j)
    if (b0 + j < nb)
      step(b0 + j, j);
  const size_t col = static_cast<size_t>(tn) * kTBN + 16 * wn + li;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const size_t row = static_cast<size_t>(tm) * kTBM + 16 * wm + 4 * q + e;
    if (row < nr && col < nc)
      s[row * bs + col] = acc[e];
  }
}

// ---- the same tiles straight from the plain rows ---------------------------
// For the reference ABI without a workspace (tcrv_hip_q8_0_q8_0_gemm,
// tcrv_hip_q4_0_q8_0_gemm) at shapes of few output tiles: each work-group packs
// its 64 weight rows and 64 tokens into records in LDS, one 8-block chunk at a
// time (a lane per row, the row's chunk span realigned as the span pack does,
// in two halves on two waves per operand), and the four
// waves fold their 32 x 32 tiles from there as gemm_tiles32 does from HBM.
// Rows 16-byte aligned and a whole number of chunks (n a multiple of 256).
constexpr int kFKB = kPackSpan;     // blocks per K chunk
constexpr int kFOp = kFKB * kTRec;  // 17408: one operand's records of a chunk
constexpr int kFStage = 2 * kFOp;   // weights then tokens

// This lane's part of a chunk: blocks 4h .. 4h + 3 of its row's span, Q8_0
// pieces 8h .. 8h + 8 (16 bytes each), Q4_0 pieces 4h .. 4h + 4.
struct Span9 {
  uint32_t v[36];
};

__device__ __forceinline__ void put_record(uint8_t *rec, int r, const uint32_t (&q)[8], uint32_t d) {
  reinterpret_cast<uint4 *>(rec)[r] = make_uint4(q[0], q[1], q[2], q[3]);
  reinterpret_cast<uint4 *>(rec + 1024)[r] = make_uint4(q[4], q[5], q[6], q[7]);
  reinterpret_cast<uint16_t *>(rec + 2048)[r] = static_cast<uint16_t>(d);
}

// Q8_0 half kH of a chunk span: block j of the half is chunk block 4kH + j at
// window byte 8kH + 34j (even j: the scale is the low half of that dword and
// the quants start 2 bytes in; odd j: the scale is the high half of the dword
// before the quants, which are dword aligned).
template <int kH>
__device__ __forceinline__ void put_q8_half(uint8_t *op, int r, const Span9 &w) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t q[8], d;
    if ((j & 1) == 0) {
      const int w0 = (8 * kH + 34 * j) / 4;
      d = w.v[w0] & 0xffffu;
#pragma unroll
      for (int m = 0; m < 8; ++m)
        q[m] = funnel16(w.v[w0 + m], w.v[w0 + m + 1]);
    } else {
      const int w0 = (8 * kH + 34 * j - 2) / 4;
      d = w.v[w0] >> 16;
#pragma unroll
      for (int m = 0; m < 8; ++m)
        q[m] = w.v[w0 + 1 + m];
    }
    put_record(op + (4 * kH + j) * kTRec, r, q, d);
  }
}

// Q4_0 half kH of a chunk span (144 bytes, block k at byte 18k): blocks 4kH ..
// 4kH + 3 from the window of pieces 4kH .. 4kH + 4 (bytes 64kH .. 64kH + 79),
// block j at window byte 8kH + 18j, its nibbles decoded to n - 8.
template <int kH>
__device__ __forceinline__ void put_q4_half(uint8_t *op, int r, const Span9 &w) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t raw[4], q[8], d;
    const int o = 8 * kH + 18 * j;
    if ((j & 1) == 0) {
      const int w0 = o / 4;
      d = w.v[w0] & 0xffffu;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        raw[m] = funnel16(w.v[w0 + m], w.v[w0 + m + 1]);
    } else {
      const int w0 = (o - 2) / 4;
      d = w.v[w0] >> 16;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        raw[m] = w.v[w0 + 1 + m];
    }
    decode_q4_quants(raw, q);
    put_record(op + (4 * kH + j) * kTRec, r, q, d);
  }
}

// The staging: a chunk's raw row spans (64 weight rows, 64 tokens, row after
// row: 272 bytes a Q8_0 span, 144 a Q4_0 one) come in by LDS DMA
// (global_load_lds_dwordx4, 64 consecutive 16-byte pieces per instruction: a
// few rows' lines each), and the lanes then read their row's span from LDS
// (b128 reads at a 272- or 144-byte stride: 16 lanes cover all 64 banks) and
// write its records.  Loading the spans straight into registers, a lane per
// row, put 64 rows' lines under every load instruction (4096 x 128 x 4096
// Q8_0: 31.0 against 27.7 us; 14336 x 128: 54.7 against 39.7; Q4_0, bound by
// its three-instruction fold, unchanged).  One raw buffer and one record
// buffer: the DMA of chunk c + 1 runs under chunk c's fold, the repack between
// two barriers.
constexpr int kFRawX8 = kTG * kFKB * kQ8Bytes;  // 17408
constexpr int kFRawX4 = kTG * kFKB * kQ4Bytes;  // 9216
constexpr int kFRawY = kTG * kFKB * kQ8Bytes;   // 17408

template <bool kQ4, int kWave>
__device__ __forceinline__ void rows_few_body(unsigned nb, float *s, const uint8_t *vx,
                                              size_t bx, const uint8_t *vy, size_t by,
                                              size_t nr, size_t nc, size_t bs, uint8_t *lds) {
  const int lane = threadIdx.x & 63;
  constexpr int wave = kWave;
  constexpr int wm = wave & 1, wn = wave >> 1;
  const int li = lane & 31, h = lane >> 5;
  const unsigned tiles_m = static_cast<unsigned>((nr + kSBM - 1) / kSBM);
  const unsigned tiles_n = static_cast<unsigned>((nc + kSBN - 1) / kSBN);
  unsigned tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const size_t m0 = static_cast<size_t>(tm) * kSBM, n0 = static_cast<size_t>(tn) * kSBN;

  constexpr int kRawX = kQ4 ? kFRawX4 : kFRawX8;
  constexpr int kXSpan = kFKB * (kQ4 ? kQ4Bytes : kQ8Bytes);  // bytes of a row's chunk
  constexpr int kYSpan = kFKB * kQ8Bytes;
  constexpr int kXPieces = kXSpan / 16, kYPieces = kYSpan / 16;  // 17 or 9; 17
  constexpr int kInst = kXPieces + kYPieces;  // DMA instructions a chunk (64 rows each operand)
  constexpr int kMine = (kInst - wave + 3) / 4;  // this wave's: instructions wave, wave + 4, ..
  uint8_t *raw = lds;                     // weights' spans, then the tokens'
  uint8_t *rec = lds + kRawX + kFRawY;    // the chunk's records: weights, then tokens

  // this lane's source of each of the wave's DMA instructions (chunk 0):
  // instruction i moves flat pieces 64m .. 64m + 63 of its operand (m = i, or
  // i - kXPieces for the tokens), row f / pieces, piece f % pieces; rows past
  // nr / nc repeat the last one (their outputs are not stored)
  const uint8_t *src[kMine];
#pragma unroll
  for (int j = 0; j < kMine; ++j) {
    const int i = wave + 4 * j;
    const bool y = i >= kXPieces;
    const int m = y ? i - kXPieces : i;
    const int pieces = y ? kYPieces : kXPieces;
    const int f = 64 * m + lane;
    const size_t row = y ? min(n0 + f / pieces, nc - 1) : min(m0 + f / pieces, nr - 1);
    src[j] = (y ? vy + row * by : vx + row * bx) + 16 * (f % pieces);
  }
  auto dma = [&](unsigned c) {
#pragma unroll
    for (int j = 0; j < kMine; ++j) {
      const int i = wave + 4 * j;
      const bool y = i >= kXPieces;
      const int m = y ? i - kXPieces : i;
      lds_void *to = (lds_void *)((char __attribute__((address_space(3))) *)raw +
                                  (y ? kRawX : 0) + 1024 * m);
      __builtin_amdgcn_global_load_lds(src[j] + static_cast<size_t>(c) * (y ? kYSpan : kXSpan),
                                       to, 16, 0, 0);
    }
  };
  // repack roles: waves 0, 1 the weight rows' halves (blocks 0-3, 4-7), waves
  // 2, 3 the tokens' halves; lane = row of the group.  A Q8_0 half is pieces
  // 8h .. 8h + 8 of the span, a Q4_0 half pieces 4h .. 4h + 4.
  constexpr bool tok = wave >= 2;
  constexpr int half = wave & 1;
  constexpr bool q4x = kQ4 && !tok;
  constexpr int kWin = q4x ? 5 : 9;  // pieces a lane reads
  auto repack = [&] {
    const uint8_t *rs = raw + (tok ? kRawX + lane * kYSpan : lane * kXSpan) +
                        (q4x ? 64 : 128) * half;
    Span9 w;
#pragma unroll
    for (int k = 0; k < kWin; ++k) {
      const uint4 x = reinterpret_cast<const uint4 *>(rs)[k];
      w.v[4 * k] = x.x; w.v[4 * k + 1] = x.y; w.v[4 * k + 2] = x.z; w.v[4 * k + 3] = x.w;
    }
    uint8_t *op = rec + (tok ? kFOp : 0);
    if constexpr (q4x)
      put_q4_half<half>(op, lane, w);
    else
      put_q8_half<half>(op, lane, w);
  };

  const uint32_t kmask = h ? 0u : 0xffffu;
  const uint32_t one = h ? 0u : 0x3c00u;
  const unsigned qa = h * 1024 + (32 * wm + li) * 16, qb = h * 1024 + (32 * wn + li) * 16;
  const unsigned sa = 2 * kTG * 16 + (32 * wm + li) * 2, sb = 2 * kTG * 16 + (32 * wn + li) * 2;
  auto ops = [&](int k) {
    const uint8_t *ra = rec + k * kTRec, *rb = ra + kFOp;
    Ops32 o;
    o.a = *reinterpret_cast<const v4i *>(ra + qa);
    o.b = *reinterpret_cast<const v4i *>(rb + qb);
    o.ux = *reinterpret_cast<const uint16_t *>(ra + sa);
    o.uy = *reinterpret_cast<const uint16_t *>(rb + sb);
    return o;
  };
  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e)
    acc[e] = 0.0f;

  const unsigned nchunks = nb / kFKB;
  dma(0);
  __builtin_amdgcn_s_waitcnt(0x070);  // this wave's DMA has landed
  __syncthreads();                     // and every wave's
  repack();
  __syncthreads();
  for (unsigned c = 0; c < nchunks; ++c) {
    const bool more = c + 1 < nchunks;
    if (more)
      dma(c + 1);  // the raw buffer: its last reader, the repack, is past a barrier
    Step32 cur = issue32<kQ4>(ops(0), kmask, one);
#pragma unroll
    for (int k = 0; k < kFKB; ++k) {
      Step32 nxt;
      if (k + 1 < kFKB)
        nxt = issue32<kQ4>(ops(k + 1), kmask, one);
      fold32<kQ4>(acc, cur);
      cur = nxt;
    }
    if (more) {
      __builtin_amdgcn_s_waitcnt(0x070);
      __syncthreads();  // every DMA landed, every wave done with the records
      repack();
      __syncthreads();
    }
  }
  store32(s, acc, m0 + 32 * wm, n0 + 32 * wn + li, h, nr, nc, bs);
}

template <bool kQ4>
__global__ __launch_bounds__(256, 2) void gemm_rows_few(unsigned nb, float *s, const uint8_t *vx,
                                                        size_t bx, const uint8_t *vy, size_t by,
                                                        size_t nr, size_t nc, size_t bs) {
  __shared__ __align__(16) uint8_t lds[kFRawX8 + kFRawY + kFStage];  // raw spans, records
  // the wave index as a template argument: each wave's staging offsets are
  // constants (as a run-time value the compiler merged the two halves' repack
  // code with the span window in scratch)
  switch (__builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6)) {
  case 0: rows_few_body<kQ4, 0>(nb, s, vx, bx, vy, by, nr, nc, bs, lds); break;
  case 1: rows_few_body<kQ4, 1>(nb, s, vx, bx, vy, by, nr, nc, bs, lds); break;
  case 2: rows_few_body<kQ4, 2>(nb, s, vx, bx, vy, by, nr, nc, bs, lds); break;
  default: rows_few_body<kQ4, 3>(nb, s, vx, bx, vy, by, nr, nc, bs, lds); break;
  }
}

}  // namespace tcrv

namespace {

constexpr bool kTiledPipe = true;
// The buffer-form DMA of the Q8_0 tiled kernels and of the 256 x 256 Q4_0
// kernel takes a K chunk's offset within a 64-row group's records as a 32-bit
// soffset: nb * kTRec must stay below 2^32 (the last 1 KB kept for the lane
// offsets), K below 63 million.  The Q8_0 entries refuse more blocks; the Q4_0
// ones run the 256 x 128 Q4_0 kernel (64-bit global_load_lds) there.
constexpr size_t kMaxTiledNb = ((static_cast<size_t>(1) << 32) - 1024) / tcrv::kTRec;

size_t tile_bytes(size_t nrows, size_t nb) {
  return (nrows + tcrv::kTG - 1) / tcrv::kTG * nb * tcrv::kTRec;
}

int pack_tiles(size_t nrows, size_t nb, const uint8_t *src, size_t bx, uint8_t *dst,
               hipStream_t st) {
  using namespace tcrv_host;
  const size_t ngroups = (nrows + tcrv::kTG - 1) / tcrv::kTG;
  size_t b0 = 0;  // blocks below b0 are packed by the span kernel
  if (aligned16(src) && (nrows == 1 || bx % 16 == 0) && nb >= tcrv::kPackSpan) {
    const size_t nspans = ngroups * (nb / tcrv::kPackSpan);
    const size_t grid = (nspans * 64 + 255) / 256;
    if (grid > 0x7fffffffu)
      return TCRV_HIP_ERR_TOO_LARGE;
    tcrv::pack_gemm_tiles_span<<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, st>>>(
        nrows, nb, src, bx, dst, nspans);
    b0 = nb / tcrv::kPackSpan * tcrv::kPackSpan;
  }
  if (b0 < nb) {
    const size_t nrec = ngroups * (nb - b0);
    const size_t grid = (nrec * 64 + 255) / 256;
    if (grid > 0x7fffffffu)
      return TCRV_HIP_ERR_TOO_LARGE;
    if (aligned4(src) && (nrows == 1 || bx % 4 == 0))
      tcrv::pack_gemm_tiles<true><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, st>>>(
          nrows, nb, src, bx, dst, b0, nrec);
    else
      tcrv::pack_gemm_tiles<false><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, st>>>(
          nrows, nb, src, bx, dst, b0, nrec);
  }
  return launch_status();
}

int pack_tiles_q4(size_t nrows, size_t nb, const uint8_t *src, size_t bx, uint8_t *dst,
                  hipStream_t st) {
  using namespace tcrv_host;
  const size_t ngroups = (nrows + tcrv::kTG - 1) / tcrv::kTG;
  size_t b0 = 0;  // blocks below b0 are packed by the span kernel
  if (aligned16(src) && (nrows == 1 || bx % 16 == 0) && nb >= tcrv::kPackSpan) {
    const size_t nspans = ngroups * (nb / tcrv::kPackSpan);
    const size_t grid = (nspans * 64 + 255) / 256;
    if (grid > 0x7fffffffu)
      return TCRV_HIP_ERR_TOO_LARGE;
    tcrv::pack_q4_tiles_span<<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, st>>>(
        nrows, nb, src, bx, dst, nspans);
    b0 = nb / tcrv::kPackSpan * tcrv::kPackSpan;
  }
  if (b0 < nb) {
    const size_t nrec = ngroups * (nb - b0);
    const size_t grid = (nrec * 64 + 255) / 256;
    if (grid > 0x7fffffffu)
      return TCRV_HIP_ERR_TOO_LARGE;
    tcrv::pack_q4_tiles<<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, st>>>(
        nrows, nb, src, bx, dst, b0, nrec);
  }
  return launch_status();
}

// Both operands of a GEMM (xq4: the weights vx are Q4_0): one launch of the span
// kernel when every block of both is in an 8-block span of 16-byte aligned rows,
// else one pack per operand.
int pack_tiles_both(size_t nb, const uint8_t *vx, size_t bx, size_t nr, uint8_t *tx,
                    const uint8_t *vy, size_t by, size_t nc, uint8_t *ty, hipStream_t st,
                    bool xq4 = false) {
  using namespace tcrv_host;
  auto spans_only = [&](const uint8_t *src, size_t stride, size_t nrows) {
    return aligned16(src) && (nrows == 1 || stride % 16 == 0) && nb % tcrv::kPackSpan == 0;
  };
  if (nb == 0 || !spans_only(vx, bx, nr) || !spans_only(vy, by, nc)) {
    const int rc = xq4 ? pack_tiles_q4(nr, nb, vx, bx, tx, st) : pack_tiles(nr, nb, vx, bx, tx, st);
    return rc != TCRV_HIP_OK ? rc : pack_tiles(nc, nb, vy, by, ty, st);
  }
  const size_t per_group = nb / tcrv::kPackSpan;
  const tcrv::SpanOperand x{vx, bx, nr, (nr + tcrv::kTG - 1) / tcrv::kTG * per_group, tx};
  const tcrv::SpanOperand y{vy, by, nc, (nc + tcrv::kTG - 1) / tcrv::kTG * per_group, ty};
  const size_t grid = ((x.nspans + y.nspans) * 64 + 255) / 256;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  if (xq4)
    tcrv::pack_gemm_tiles_span2<true>
        <<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, st>>>(nb, x, y);
  else
    tcrv::pack_gemm_tiles_span2<false>
        <<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, st>>>(nb, x, y);
  return launch_status();
}

// Which Q8_0 kernel serves a shape: both fold every output in the same order, so
// the choice is speed only.  One MI355X runs 256 work-groups of either kernel at
// once (one per CU); a round of 256 x 256 tiles takes ~1.87 times a round of
// 256 x 128 ones at equal K (4096^3: one round 150-152 us against two rounds in
// 161 us), and a lone round of the smaller tile 93 us.  So the larger tile runs
// when its rounds x 15 are at most the smaller tile's rounds x 8: at 4096 x 4096
// outputs (one round against two) and at 8192 x 4096 (two against four), not at
// 4096 x 2048 (half the CUs idle) or 4196 x 4166 (two against three).
bool tiles256_first(size_t tiles, size_t tiles256) {
  constexpr size_t kCUs = 256;
  return (tiles256 + kCUs - 1) / kCUs * 15 <= (tiles + kCUs - 1) / kCUs * 8;
}

// Few work-group tiles: the one-tile-a-wave kernel where the 256 x 128 tiles
// would not fill one round of the CUs and its own waves fit two rounds of two
// a SIMD (at most 1024 work-groups).  Pre-packed operands, K 4096 unless
// named, us, 256 x 128 tiles against it: 4096 x 128 72 / 17, 4096 x 512 74 /
// 28, 4096 x 1024 75 / 53, 14336 x 128 72 / 27, 4096 x 128 x 14336 234 / 51;
// but 14336 x 512 (1792 of its work-groups) 82 / 88, and from 256 tiles (a
// full round) the larger tiles win: 4096 x 2048 93-98 against ~100.
bool tiles32_first(size_t tiles, size_t tiles64, size_t nb) {
  return tiles < 256 && tiles64 <= 1024 && nb <= 0xffffffffu;
}

// Fewer still: one 16 x 16 tile a wave while its waves fit one a SIMD (at most
// 256 work-groups of 32 x 32).  Pre-packed, K 4096, us, 32 x 32 tiles against
// it: 4096 x 2 17.0 / 13.1, 4096 x 64 17.1 / 13.7 (Q4_0 19.8 / 14.9); past
// that its loads and doubled VALU per output lose (4096 x 128: 17.5 / 24.2).
bool tiles16_first(size_t nr, size_t nc) {
  return ((nr + tcrv::kTBM - 1) / tcrv::kTBM) * ((nc + tcrv::kTBN - 1) / tcrv::kTBN) <= 256;
}

size_t tiles64_of(size_t nr, size_t nc) {
  return ((nr + tcrv::kSBM - 1) / tcrv::kSBM) * ((nc + tcrv::kSBN - 1) / tcrv::kSBN);
}
size_t tiles128_of(size_t nr, size_t nc) {
  return ((nr + tcrv::kDBM - 1) / tcrv::kDBM) * ((nc + tcrv::kDBN - 1) / tcrv::kDBN);
}

int gemm_tiles(size_t nb, float *s, const uint8_t *tx, const uint8_t *ty, size_t nr, size_t nc,
               size_t bs, hipStream_t st, bool q4 = false) {
  using namespace tcrv_host;
  const size_t tiles = ((nr + tcrv::kDBM - 1) / tcrv::kDBM) * ((nc + tcrv::kDBN - 1) / tcrv::kDBN);
  if (tiles > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  const size_t tiles256 =
      ((nr + tcrv::kEBM - 1) / tcrv::kEBM) * ((nc + tcrv::kEBN - 1) / tcrv::kEBN);
  const size_t tiles64 =
      ((nr + tcrv::kSBM - 1) / tcrv::kSBM) * ((nc + tcrv::kSBN - 1) / tcrv::kSBN);
  if (tiles32_first(tiles, tiles64, nb) && tiles16_first(nr, nc)) {
    const size_t tiles32n =
        ((nr + tcrv::kTBM - 1) / tcrv::kTBM) * ((nc + tcrv::kTBN - 1) / tcrv::kTBN);
    const unsigned nbu = static_cast<unsigned>(nb);
    if (q4)
      tcrv::gemm_tiles16<true><<<dim3(static_cast<unsigned>(tiles32n)), dim3(256), 0, st>>>(
          nbu, s, tx, ty, nr, nc, bs);
    else
      tcrv::gemm_tiles16<false><<<dim3(static_cast<unsigned>(tiles32n)), dim3(256), 0, st>>>(
          nbu, s, tx, ty, nr, nc, bs);
  } else if (tiles32_first(tiles, tiles64, nb)) {
    const unsigned nbu = static_cast<unsigned>(nb);
    if (q4)
      tcrv::gemm_tiles32<true><<<dim3(static_cast<unsigned>(tiles64)), dim3(256), 0, st>>>(
          nbu, s, tx, ty, nr, nc, bs);
    else
      tcrv::gemm_tiles32<false><<<dim3(static_cast<unsigned>(tiles64)), dim3(256), 0, st>>>(
          nbu, s, tx, ty, nr, nc, bs);
  } else if (q4 && nb <= kMaxTiledNb && tiles256_first(tiles, tiles256))
    tcrv::gemm_tiles256_q4<<<dim3(static_cast<unsigned>(tiles256)), dim3(tcrv::kEThreads), 0,
                             st>>>(nb, s, tx, ty, nr, nc, bs);
  else if (q4)
    tcrv::gemm_tiles_q4<<<dim3(static_cast<unsigned>(tiles)), dim3(tcrv::kDThreads), 0, st>>>(
        nb, s, tx, ty, nr, nc, bs);
  else if (tiles256_first(tiles, tiles256))
    tcrv::gemm_tiles256_q8<<<dim3(static_cast<unsigned>(tiles256)), dim3(tcrv::kEThreads), 0,
                             st>>>(nb, s, tx, ty, nr, nc, bs);
  else
    tcrv::gemm_tiles_q8<kTiledPipe><<<dim3(static_cast<unsigned>(tiles)),
                                      dim3(tcrv::kDThreads), 0, st>>>(nb, s, tx, ty, nr, nc, bs);
  return launch_status();
}

}  // namespace

extern "C" {

size_t tcrv_hip_gemm_tiles_bytes(size_t nrows, size_t nb) { return tile_bytes(nrows, nb); }

int tcrv_hip_pack_q8_0_to_gemm_tiles(size_t nrows, size_t nb, const uint8_t *src, size_t bx,
                                     uint8_t *dst, void *stream) {
  using namespace tcrv_host;
  if (nrows == 0 || nb == 0)
    return TCRV_HIP_OK;
  if (!src || !dst)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(src) || (nrows > 1 && (bx & 1u)) || !aligned16(dst))
    return TCRV_HIP_ERR_MISALIGNED;
  if (nrows > 1 && bx < nb * tcrv::kQ8Bytes)
    return TCRV_HIP_ERR_BAD_SIZE;
  return pack_tiles(nrows, nb, src, bx, dst, as_stream(stream));
}

int tcrv_hip_q8_0_q8_0_gemm_tiles(size_t n, float *s, const uint8_t *tx, const uint8_t *ty,
                                  size_t nr, size_t nc, size_t bs, void *stream) {
  using namespace tcrv_host;
  const size_t nb = n / tcrv::kQK;
  if (nr == 0 || nc == 0)
    return TCRV_HIP_OK;
  if (nr > 1 && bs < nc)
    return TCRV_HIP_ERR_BAD_SIZE;
  if (nb == 0)
    return zero_outputs(s, nr * nc, bs, nc, stream);
  if (nb > kMaxTiledNb)
    return TCRV_HIP_ERR_TOO_LARGE;
  if (!s || !tx || !ty)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned16(tx) || !aligned16(ty))
    return TCRV_HIP_ERR_MISALIGNED;
  return gemm_tiles(nb, s, tx, ty, nr, nc, bs, as_stream(stream));
}

}  // extern "C"

namespace tcrv_host {

// The plain-row entries' kernel for shapes of few output tiles (gemm_rows_few):
// rows 16-byte aligned, a whole number of 8-block chunks, the shapes
// gemm_tiles32 serves (at its 1024 work-groups the 256-row kernels are as fast:
// 4096 x 1024 x 4096 Q8_0 91.6 against 91-93 us).
int gemm_rows_few(bool q4, size_t nb, float *s, const uint8_t *vx, size_t bx, const uint8_t *vy,
                  size_t by, size_t nr, size_t nc, size_t bs, void *stream) {
  if (nr < 2 || nc < 2 || nb == 0 || nb % tcrv::kFKB != 0 || !aligned16(vx) || !aligned16(vy) ||
      bx % 16 != 0 || by % 16 != 0)
    return TCRV_HIP_ERR_UNSUPPORTED;
  const size_t tiles64 = tiles64_of(nr, nc);
  if (!tiles32_first(tiles128_of(nr, nc), tiles64, nb))
    return TCRV_HIP_ERR_UNSUPPORTED;
  const dim3 g(static_cast<unsigned>(tiles64)), b(256);
  const unsigned nbu = static_cast<unsigned>(nb);
  if (q4)
    tcrv::gemm_rows_few<true><<<g, b, 0, as_stream(stream)>>>(nbu, s, vx, bx, vy, by, nr, nc, bs);
  else
    tcrv::gemm_rows_few<false><<<g, b, 0, as_stream(stream)>>>(nbu, s, vx, bx, vy, by, nr, nc, bs);
  return launch_status();
}

// Shapes the tiled kernel does not serve run as tcrv_hip_q8_0_q8_0_gemm,
// without the workspace: fewer weight rows than one 256-row tile, a single
// token (decode), no blocks, or more than kMaxTiledNb blocks.  So do a few
// tokens that the plain entry's multi-column GEMVs take (even block count,
// 4-byte aligned rows and strides; cols_first): there they beat packing both
// operands for the tiled kernels (us, 4096 weight rows, K 4096, Q8_0 / Q4_0:
// 16 tokens 15.0 / 16.3 against ~25 / ~28; 32 tokens 30.8 / 32.3 against
// 23.9 / 26.9).
bool ws_cols_first(size_t nb, const uint8_t *vx, size_t bx, const uint8_t *vy, size_t by,
                   size_t nr, size_t nc) {
  return cols_first(nr, nc) && nb % 2 == 0 && aligned4(vx) && aligned4(vy) && bx % 4 == 0 &&
         by % 4 == 0;
}
// And where the plain entry's few-tile kernel, which packs in LDS, beats a
// separate pack: up to 448 of its work-groups at K up to 4096, past the 16 x 16
// tiles' shapes (us, plain against the workspace path: 4096 x 128 x 4096 28.0 /
// 30.6 Q8_0, 31.5 / 32.2 Q4_0; 14336 x 128 40.7 / 48.7, 42.0 / 45.9; but 4096 x
// 512 41.8 / 39.9, 4096 x 128 x 14336 84.1 / 72.5).
bool ws_rows_few_first(size_t nb, const uint8_t *vx, size_t bx, const uint8_t *vy, size_t by,
                       size_t nr, size_t nc) {
  return nb % tcrv::kFKB == 0 && nb <= 128 && aligned16(vx) && aligned16(vy) && bx % 16 == 0 &&
         by % 16 == 0 && tiles32_first(tiles128_of(nr, nc), tiles64_of(nr, nc), nb) &&
         !tiles16_first(nr, nc) && tiles64_of(nr, nc) <= 448;
}

bool gemm_ws_uses_workspace(size_t n, const uint8_t *vx, size_t bx, const uint8_t *vy,
                            size_t by, size_t nr, size_t nc) {
  const size_t nb = n / tcrv::kQK;
  return nr >= static_cast<size_t>(tcrv::kDBM) && nc >= 2 && nb > 0 && nb <= kMaxTiledNb &&
         !ws_cols_first(nb, vx, bx, vy, by, nr, nc) &&
         !ws_rows_few_first(nb, vx, bx, vy, by, nr, nc);
}

}  // namespace tcrv_host

extern "C" {

size_t tcrv_hip_q8_0_q8_0_gemm_workspace_bytes(size_t n, size_t nr, size_t nc) {
  const size_t nb = n / tcrv::kQK;
  return tile_bytes(nr, nb) + tile_bytes(nc, nb);
}

int tcrv_hip_q8_0_q8_0_gemm_ws(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                               size_t by, size_t nr, size_t nc, size_t bx, size_t bs,
                               void *workspace, size_t workspace_bytes, void *stream) {
  using namespace tcrv_host;
  const size_t nb = n / tcrv::kQK;
  if (!gemm_ws_uses_workspace(n, vx, bx, vy, by, nr, nc))
    return tcrv_hip_q8_0_q8_0_gemm(n, s, vx, vy, by, nr, nc, bx, bs, stream);
  if (bs < nc)
    return TCRV_HIP_ERR_BAD_SIZE;
  if (!s || !vx || !vy || !workspace)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(vx) || !aligned2(vy) || (bx & 1u) || (by & 1u) || !aligned16(workspace))
    return TCRV_HIP_ERR_MISALIGNED;
  const size_t rowbytes = nb * tcrv::kQ8Bytes;
  if (bx < rowbytes || by < rowbytes)
    return TCRV_HIP_ERR_BAD_SIZE;
  const size_t tx_bytes = tile_bytes(nr, nb), ty_bytes = tile_bytes(nc, nb);
  if (workspace_bytes < tx_bytes + ty_bytes)
    return TCRV_HIP_ERR_BAD_SIZE;
  uint8_t *tx = static_cast<uint8_t *>(workspace);
  uint8_t *ty = tx + tx_bytes;  // tx_bytes is a multiple of 2176 = 16 * 136
  hipStream_t st = as_stream(stream);
  const int rc = pack_tiles_both(nb, vx, bx, nr, tx, vy, by, nc, ty, st);
  if (rc != TCRV_HIP_OK)
    return rc;
  return gemm_tiles(nb, s, tx, ty, nr, nc, bs, st);
}

int tcrv_hip_pack_q4_0_to_gemm_tiles(size_t nrows, size_t nb, const uint8_t *src, size_t bx,
                                     uint8_t *dst, void *stream) {
  using namespace tcrv_host;
  if (nrows == 0 || nb == 0)
    return TCRV_HIP_OK;
  if (!src || !dst)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(src) || (nrows > 1 && (bx & 1u)) || !aligned16(dst))
    return TCRV_HIP_ERR_MISALIGNED;
  if (nrows > 1 && bx < nb * tcrv::kQ4Bytes)
    return TCRV_HIP_ERR_BAD_SIZE;
  return pack_tiles_q4(nrows, nb, src, bx, dst, as_stream(stream));
}

int tcrv_hip_q4_0_q8_0_gemm_tiles(size_t n, float *s, const uint8_t *tx, const uint8_t *ty,
                                  size_t nr, size_t nc, size_t bs, void *stream) {
  using namespace tcrv_host;
  const size_t nb = n / tcrv::kQK;
  if (nr == 0 || nc == 0)
    return TCRV_HIP_OK;
  if (nr > 1 && bs < nc)
    return TCRV_HIP_ERR_BAD_SIZE;
  if (nb == 0)
    return zero_outputs(s, nr * nc, bs, nc, stream);
  if (!s || !tx || !ty)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned16(tx) || !aligned16(ty))
    return TCRV_HIP_ERR_MISALIGNED;
  return gemm_tiles(nb, s, tx, ty, nr, nc, bs, as_stream(stream), true);
}

size_t tcrv_hip_q4_0_q8_0_gemm_workspace_bytes(size_t n, size_t nr, size_t nc) {
  const size_t nb = n / tcrv::kQK;
  return tile_bytes(nr, nb) + tile_bytes(nc, nb);
}

int tcrv_hip_q4_0_q8_0_gemm_ws(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                               size_t by, size_t nr, size_t nc, size_t bx, size_t bs,
                               void *workspace, size_t workspace_bytes, void *stream) {
  using namespace tcrv_host;
  const size_t nb = n / tcrv::kQK;
  if (!gemm_ws_uses_workspace(n, vx, bx, vy, by, nr, nc))
    return tcrv_hip_q4_0_q8_0_gemm(n, s, vx, vy, by, nr, nc, bx, bs, stream);
  if (bs < nc)
    return TCRV_HIP_ERR_BAD_SIZE;
  if (!s || !vx || !vy || !workspace)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(vx) || !aligned2(vy) || (bx & 1u) || (by & 1u) || !aligned16(workspace))
    return TCRV_HIP_ERR_MISALIGNED;
  if (bx < nb * tcrv::kQ4Bytes || by < nb * tcrv::kQ8Bytes)
    return TCRV_HIP_ERR_BAD_SIZE;
  const size_t tx_bytes = tile_bytes(nr, nb), ty_bytes = tile_bytes(nc, nb);
  if (workspace_bytes < tx_bytes + ty_bytes)
    return TCRV_HIP_ERR_BAD_SIZE;
  uint8_t *tx = static_cast<uint8_t *>(workspace);
  uint8_t *ty = tx + tx_bytes;  // tx_bytes is a multiple of 2176 = 16 * 136
  hipStream_t st = as_stream(stream);
  const int rc = pack_tiles_both(nb, vx, bx, nr, tx, vy, by, nc, ty, st, true);
  if (rc != TCRV_HIP_OK)
    return rc;
  return gemm_tiles(nb, s, tx, ty, nr, nc, bs, st, true);
}

}  // extern "C"
