// Device scratch of the entry point that allocates nothing
// (tfd_laya_attention_block_noalloc_f32, declared in tfd_attention.h): one
// file-scope array per GPU, loaded with the library's code object and held
// until the process ends. Host code never passes the array's name to a
// kernel: it asks noalloc_scratch() for the array's address on the current
// device, looked up once per device with hipGetSymbolAddress.
#include <mutex>

#include "tfd_internal.hpp"

namespace tfd {

static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_lock;
void *g_scratch[kMaxDevices];  // the array's address on each device, once looked up
}  // namespace

void *noalloc_scratch(int device, hipError_t *err) {
  *err = hipSuccess;
  if (device < 0 || device >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> guard(g_lock);
  if (g_scratch[device] == nullptr) {
    // The caller has made `device` current: each GPU holds its own copy of
    // the array at its own address.
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
      return nullptr;
    }
    g_scratch[device] = p;
  }
  return g_scratch[device];
}

}  // namespace tfd
