// Slab state pool: slot bookkeeping over a caller-allocated slab of equal fp32 state slots.
//
// The recurrent slab of the reference's HybridMemoryPool (serving/hybrid_memory_pool.{h,cpp}): a free-slot
// stack handing out the lowest free slot first (hybrid_memory_pool.cpp:30-37, 50-60), fork as a device
// copy of the parent's slot into a new one (:86-116), release back onto the stack (:118-135), and the
// allocated / free byte accounting (:137-147).  The slab itself belongs to the caller (any device
// allocation, e.g. a torch tensor), so the pool allocates no device memory; a new slot is zeroed on the
// device, as the reference's torch pool starts from zeros (serving/vllm_hybrid_model_runner.py:40-44).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <new>
#include <vector>
#include "kdn_internal.hpp"

struct kdn_pool {
  int64_t max_slots = 0, slot_bytes = 0;
  std::vector<int32_t> free_stack;  // top = back(); initialised so that slot 0 is handed out first
  std::vector<uint8_t> active;
};

namespace kdn {

// Zero `n16` 16-byte words (vector stores).
__global__ void __launch_bounds__(256) zero_kernel(uint4* __restrict__ dst, int64_t n16) {
  const uint4 z = {0u, 0u, 0u, 0u};
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256) dst[i] = z;
}

static int zero_slot(void* base, int64_t bytes, hipStream_t st) {
  const int64_t n16 = bytes / 16;
  int64_t blocks = (n16 + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (uint4*)base, n16);
  return launch_status();
}

static bool is_active(const kdn_pool* p, int slot) {
  return p && slot >= 0 && slot < p->max_slots && p->active[(size_t)slot];
}

}  // namespace kdn

using namespace kdn;

extern "C" int kdn_pool_create(int64_t max_slots, int64_t slot_bytes, kdn_pool** out) {
  if (!out) return KDN_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  if (max_slots <= 0 || max_slots > INT32_MAX || slot_bytes <= 0 || slot_bytes % 16 != 0) return KDN_ERR_INVALID_ARGUMENT;
  kdn_pool* p = new (std::nothrow) kdn_pool;
  if (!p) return KDN_ERR_CAPACITY;
  p->max_slots = max_slots;
  p->slot_bytes = slot_bytes;
  p->free_stack.reserve((size_t)max_slots);
  for (int64_t i = max_slots - 1; i >= 0; --i) p->free_stack.push_back((int32_t)i);
  p->active.assign((size_t)max_slots, 0);
  *out = p;
  return KDN_OK;
}

extern "C" void kdn_pool_destroy(kdn_pool* pool) { delete pool; }

extern "C" int kdn_pool_allocate(kdn_pool* pool, void* slab, void* stream) {
  if (!pool) return KDN_ERR_INVALID_ARGUMENT;
  if (slab && !aligned(slab, 16)) return KDN_ERR_MISALIGNED;
  if (pool->free_stack.empty()) return KDN_ERR_CAPACITY;
  const int32_t slot = pool->free_stack.back();
  if (slab) {
    const int rc = zero_slot((unsigned char*)slab + (size_t)slot * (size_t)pool->slot_bytes, pool->slot_bytes,
                             as_stream(stream));
    if (rc != KDN_OK) return rc;
  }
  pool->free_stack.pop_back();
  pool->active[(size_t)slot] = 1;
  return slot;
}

extern "C" int kdn_pool_fork(kdn_pool* pool, int parent, void* slab, void* stream) {
  if (!is_active(pool, parent)) return KDN_ERR_INVALID_ARGUMENT;
  if (pool->free_stack.empty()) return KDN_ERR_CAPACITY;
  const int32_t child = pool->free_stack.back();
  if (slab) {
    unsigned char* base = (unsigned char*)slab;
    const size_t sb = (size_t)pool->slot_bytes;
    if (hipMemcpyAsync(base + (size_t)child * sb, base + (size_t)parent * sb, sb, hipMemcpyDeviceToDevice,
                       as_stream(stream)) != hipSuccess)
      return KDN_ERR_DEVICE;
  }
  pool->free_stack.pop_back();
  pool->active[(size_t)child] = 1;
  return child;
}

extern "C" int kdn_pool_release(kdn_pool* pool, int slot) {
  if (!is_active(pool, slot)) return KDN_ERR_INVALID_ARGUMENT;
  pool->active[(size_t)slot] = 0;
  pool->free_stack.push_back((int32_t)slot);
  return KDN_OK;
}

extern "C" int64_t kdn_pool_active(const kdn_pool* pool) {
  return pool ? pool->max_slots - (int64_t)pool->free_stack.size() : 0;
}

extern "C" int64_t kdn_pool_allocated_bytes(const kdn_pool* pool) {
  return pool ? kdn_pool_active(pool) * pool->slot_bytes : 0;
}

extern "C" int64_t kdn_pool_free_bytes(const kdn_pool* pool) {
  return pool ? (int64_t)pool->free_stack.size() * pool->slot_bytes : 0;
}
