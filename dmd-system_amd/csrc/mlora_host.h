// Host-side validation shared by the C-ABI entry points: every check runs
// before any launch, so a bad call returns an error code and enqueues nothing.
#pragma once

#include <stdint.h>

#include "mlora_common.h"

namespace mlora {

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Copy and validate the routing arrays (seg_offsets int64 [n+1], adapter_ids [n]).
inline int build_segtable(SegTable &st, int64_t M, const int64_t *off, const int32_t *aid, int32_t n,
                          int32_t n_adapters) {
  if (off == nullptr || aid == nullptr || n < 1 || M < 0) return MLORA_ERR_INVALID;
  if (n > kMaxSeg) return MLORA_ERR_LIMIT;
  if (M > (int64_t)INT32_MAX - 1024) return MLORA_ERR_LIMIT;
  if (off[0] != 0 || off[n] != M) return MLORA_ERR_INVALID;
  st.n = n;
  for (int s = 0; s < n; ++s) {
    if (off[s + 1] < off[s]) return MLORA_ERR_INVALID;
    if (aid[s] < -1 || aid[s] >= n_adapters) return MLORA_ERR_INVALID;
    st.off[s] = (int32_t)off[s];
    st.aid[s] = aid[s];
  }
  st.off[n] = (int32_t)M;
  return MLORA_OK;
}

// True if adapter a owns at least one row.
inline bool adapter_used(const SegTable &st, int a) {
  for (int s = 0; s < st.n; ++s)
    if (st.aid[s] == a && st.off[s + 1] > st.off[s]) return true;
  return false;
}

// Validate the adapter table. A used adapter with rank > 0 needs a 16-byte
// aligned operand pointer; ranks are 0 or multiples of 8 in [8, max_rank] (kMaxRank, or
// kMaxGemmRank for the GEMMs, whose LoRA term is any number of extra k-tiles).
inline int build_adapters(AdapterTable &at, const SegTable &st, const void *const *ptrs, const int32_t *ranks,
                          const float *scales, int32_t n, int32_t max_rank = kMaxRank) {
  if (n < 0) return MLORA_ERR_INVALID;
  if (n > kMaxAdapters) return MLORA_ERR_LIMIT;
  if (n > 0 && ranks == nullptr) return MLORA_ERR_INVALID;
  for (int a = 0; a < kMaxAdapters; ++a) {
    at.ptr[a] = nullptr;
    at.rank[a] = 0;
    at.scale[a] = 0.f;
  }
  for (int a = 0; a < n; ++a) {
    const int r = ranks[a];
    if (r < 0 || (r > 0 && r < 8) || (r % 8) != 0) return r > max_rank ? MLORA_ERR_LIMIT : MLORA_ERR_INVALID;
    if (r > max_rank) return MLORA_ERR_LIMIT;
    at.rank[a] = r;
    at.scale[a] = scales ? scales[a] : 1.f;
    if (r > 0 && adapter_used(st, a)) {
      if (ptrs == nullptr || ptrs[a] == nullptr) return MLORA_ERR_INVALID;
      if (!aligned16(ptrs[a])) return MLORA_ERR_UNSUPPORTED;
      at.ptr[a] = static_cast<const uint16_t *>(ptrs[a]);
    }
  }
  return MLORA_OK;
}

// Largest rank among adapters that own rows.
inline int max_used_rank(const SegTable &st, const AdapterTable &at) {
  int r = 0;
  for (int s = 0; s < st.n; ++s) {
    const int a = st.aid[s];
    if (a >= 0 && st.off[s + 1] > st.off[s] && at.rank[a] > r) r = at.rank[a];
  }
  return r;
}

// bf16 row-major matrix [rows, cols] with leading dimension ld: pointer and
// stride must allow 16-byte vector access of 8-element chunks.
inline int check_bf16_matrix(const void *p, int64_t ld, int64_t rows, int64_t cols) {
  if (rows == 0 || cols == 0) return MLORA_OK;
  if (p == nullptr || ld < cols) return MLORA_ERR_INVALID;
  if (!aligned16(p) || (ld % 8) != 0 || (cols % 8) != 0) return MLORA_ERR_UNSUPPORTED;
  return MLORA_OK;
}

// e4m3 matrices: rows of 16-byte chunks (ld and cols multiples of 16).
inline int check_fp8_matrix(const void *p, int64_t ld, int64_t rows, int64_t cols) {
  if (rows == 0 || cols == 0) return MLORA_OK;
  if (p == nullptr || ld < cols) return MLORA_ERR_INVALID;
  if (!aligned16(p) || (ld % 16) != 0 || (cols % 16) != 0) return MLORA_ERR_UNSUPPORTED;
  return MLORA_OK;
}

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLORA_OK : MLORA_ERR_LAUNCH;
}

}  // namespace mlora
