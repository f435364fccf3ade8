// block_pq4 / block_pq2 layout constants, shared by host and device code.
#pragma once

#ifdef __HIPCC__
#define PQKV_HD __host__ __device__
#else
#define PQKV_HD
#endif

namespace pqkv {

constexpr int kBlock = 32;            // coordinates per block
constexpr int kPq4BlockBytes = 18;    // {fp16 d; u8 qs[16]}
constexpr int kPq2BlockBytes = 10;    // {fp16 d; u8 qs[8]}

PQKV_HD constexpr int block_bytes(int bits) { return bits == 4 ? kPq4BlockBytes : kPq2BlockBytes; }
PQKV_HD constexpr int vector_bytes(int d, int bits) { return (d / kBlock) * block_bytes(bits); }
// Byte offset, inside one vector, of qs byte p (p counts packed bytes over the
// whole vector: 16 per block for 4-bit codes, 8 per block for 2-bit codes).
PQKV_HD constexpr int qs_offset(int p, int bits) {
  return bits == 4 ? (p >> 4) * kPq4BlockBytes + 2 + (p & 15) : (p >> 3) * kPq2BlockBytes + 2 + (p & 7);
}

}  // namespace pqkv
