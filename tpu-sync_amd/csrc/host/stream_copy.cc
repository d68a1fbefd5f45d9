#include "stream_copy.h"

#include <immintrin.h>

#include <cstdint>
#include <cstring>

namespace kvx {
namespace {

// 16-byte streaming stores: SSE2 is part of x86-64, so this body always runs.
void StreamBody16(uint8_t* d, const uint8_t* s, size_t n) {
  for (size_t i = 0; i < n; i += 64) {
    const __m128i a = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i));
    const __m128i b = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i + 16));
    const __m128i c = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i + 32));
    const __m128i e = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i + 48));
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i), a);
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i + 16), b);
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i + 32), c);
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i + 48), e);
  }
}

// 32-byte streaming stores, two cache lines per iteration.
__attribute__((target("avx2"))) void StreamBody32(uint8_t* d, const uint8_t* s, size_t n) {
  for (size_t i = 0; i < n; i += 128) {
    const __m256i a = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(s + i));
    const __m256i b = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(s + i + 32));
    const __m256i c = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(s + i + 64));
    const __m256i e = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(s + i + 96));
    _mm256_stream_si256(reinterpret_cast<__m256i*>(d + i), a);
    _mm256_stream_si256(reinterpret_cast<__m256i*>(d + i + 32), b);
    _mm256_stream_si256(reinterpret_cast<__m256i*>(d + i + 64), c);
    _mm256_stream_si256(reinterpret_cast<__m256i*>(d + i + 96), e);
  }
}

// A build may fix the choice (the CPU test builds both bodies this way).
#ifndef KVX_STREAM_COPY_AVX2
#define KVX_STREAM_COPY_AVX2 __builtin_cpu_supports("avx2")
#endif
const bool g_avx2 = KVX_STREAM_COPY_AVX2;

}  // namespace

void StreamCopy(void* dst, const void* src, size_t bytes) {
  if (bytes < kStreamCopyMinBytes) {
    std::memcpy(dst, src, bytes);
    return;
  }
  uint8_t* d = static_cast<uint8_t*>(dst);
  const uint8_t* s = static_cast<const uint8_t*>(src);
  // Head up to the first 64-byte boundary of the destination (streaming
  // stores need aligned addresses), a body of whole 128-byte steps, and the
  // tail, both with memcpy.
  const size_t head = (64 - (reinterpret_cast<uintptr_t>(d) & 63)) & 63;
  std::memcpy(d, s, head);
  const size_t body = (bytes - head) & ~static_cast<size_t>(127);
  if (g_avx2) {
    StreamBody32(d + head, s + head, body);
  } else {
    StreamBody16(d + head, s + head, body);
  }
  std::memcpy(d + head + body, s + head + body, bytes - head - body);
}

void StreamFence() { _mm_sfence(); }

void PrefetchSource(const void* src, size_t bytes) {
  const char* s = static_cast<const char*>(src);
  const size_t n = bytes < kPrefetchBytes ? bytes : kPrefetchBytes;
  for (size_t o = 0; o < n; o += 64) _mm_prefetch(s + o, _MM_HINT_T0);
}

}  // namespace kvx
