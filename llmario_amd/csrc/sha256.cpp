// sha256.cpp — the SHA-256 compression function (FIPS 180-4 §6.2.2) for the prefix-cache hash
// chain: portable scalar code, and the x86 SHA extensions (SHA256RNDS2 / SHA256MSG1 / SHA256MSG2)
// when the host CPU reports them, chosen once at run time. Host code only.
#include <stddef.h>
#include <stdint.h>

#include <immintrin.h>

#include "pool.h"

namespace lmh {
namespace {

alignas(16) const uint32_t K256[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

void compress_scalar(uint32_t st[8], const uint8_t* p, size_t blocks) {
  for (; blocks > 0; blocks--, p += 64) {
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
      w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
    for (int i = 16; i < 64; i++) {
      const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = st[0], b = st[1], c = st[2], d = st[3], e = st[4], f = st[5], g = st[6], h = st[7];
    for (int i = 0; i < 64; i++) {
      const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K256[i] + w[i];
      const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
      h = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    st[0] += a;
    st[1] += b;
    st[2] += c;
    st[3] += d;
    st[4] += e;
    st[5] += f;
    st[6] += g;
    st[7] += h;
  }
}

// The SHA extensions keep the state as two vectors, (A, B, E, F) and (C, D, G, H), and run two
// rounds per SHA256RNDS2 with the message-plus-constant words in the low half of its third
// operand. Message words 4i..4i+3 for i >= 4 come from the previous sixteen through
// SHA256MSG1 (the sigma0 terms), an add of words t-7 and SHA256MSG2 (the sigma1 terms).
__attribute__((target("sha,sse4.1,ssse3"))) void compress_shani(uint32_t st[8], const uint8_t* p, size_t blocks) {
  const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bULL, 0x0405060700010203ULL);
  __m128i dcba = _mm_loadu_si128((const __m128i*)&st[0]);
  __m128i hgfe = _mm_loadu_si128((const __m128i*)&st[4]);
  __m128i cdab = _mm_shuffle_epi32(dcba, 0xB1);
  __m128i efgh = _mm_shuffle_epi32(hgfe, 0x1B);
  __m128i abef = _mm_alignr_epi8(cdab, efgh, 8);
  __m128i cdgh = _mm_blend_epi16(efgh, cdab, 0xF0);
  for (; blocks > 0; blocks--, p += 64) {
    const __m128i abef0 = abef, cdgh0 = cdgh;
    __m128i w[4];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      __m128i wi;
      if (i < 4) {
        wi = _mm_shuffle_epi8(_mm_loadu_si128((const __m128i*)(p + 16 * i)), bswap);
      } else {
        wi = _mm_sha256msg1_epu32(w[i & 3], w[(i + 1) & 3]);
        wi = _mm_add_epi32(wi, _mm_alignr_epi8(w[(i + 3) & 3], w[(i + 2) & 3], 4));
        wi = _mm_sha256msg2_epu32(wi, w[(i + 3) & 3]);
      }
      w[i & 3] = wi;
      __m128i m = _mm_add_epi32(wi, _mm_load_si128((const __m128i*)&K256[4 * i]));
      cdgh = _mm_sha256rnds2_epu32(cdgh, abef, m);
      m = _mm_shuffle_epi32(m, 0x0E);
      abef = _mm_sha256rnds2_epu32(abef, cdgh, m);
    }
    abef = _mm_add_epi32(abef, abef0);
    cdgh = _mm_add_epi32(cdgh, cdgh0);
  }
  const __m128i feba = _mm_shuffle_epi32(abef, 0x1B);
  const __m128i dchg = _mm_shuffle_epi32(cdgh, 0xB1);
  _mm_storeu_si128((__m128i*)&st[0], _mm_blend_epi16(feba, dchg, 0xF0));
  _mm_storeu_si128((__m128i*)&st[4], _mm_alignr_epi8(dchg, feba, 8));
}

using CompressFn = void (*)(uint32_t*, const uint8_t*, size_t);

CompressFn pick() {
  __builtin_cpu_init();
  if (__builtin_cpu_supports("sha") && __builtin_cpu_supports("sse4.1") && __builtin_cpu_supports("ssse3"))
    return compress_shani;
  return compress_scalar;
}

const CompressFn g_compress = pick();

}  // namespace

void sha256_compress(uint32_t state[8], const uint8_t* data, size_t blocks) { g_compress(state, data, blocks); }

// Test hook: run the scalar path (path 0) or the SHA-extension path (path 1) directly; returns false
// if that path is not available on this host.
bool sha256_compress_path(int path, uint32_t state[8], const uint8_t* data, size_t blocks) {
  if (path == 0) {
    compress_scalar(state, data, blocks);
    return true;
  }
  if (pick() != compress_shani) return false;
  compress_shani(state, data, blocks);
  return true;
}

}  // namespace lmh
