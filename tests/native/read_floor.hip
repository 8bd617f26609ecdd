// Read floor of the decode shapes: the time a plain streaming read of a
// given number of bytes takes on this GPU, measured the way bench.py times
// the library (HIP-graph replays of back-to-back launches, each launch
// reading its own buffer, buffers rotated over more than 512 MB so every
// launch reads HBM).  Also the in-graph cost of an empty launch.
//
// Usage: read_floor BYTES [BYTES ...]
// Prints one JSON object per line: {"bytes": B, "us": median, "us_min": m,
// "GBps": B / median}, then {"empty_launch_us": ...}.
//
// The read kernel: a grid-stride loop of 16-byte loads, four independent
// loads in flight per thread per iteration, 2048 workgroups of 256 threads
// at most (fewer for small buffers, at least 4 loads per thread), the loaded
// words XOR-folded into one value that is stored only if it equals a value
// the host never passes (so the loads cannot be removed).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <vector>

#define CK(x)                                                                       \
  do {                                                                              \
    hipError_t e_ = (x);                                                            \
    if (e_ != hipSuccess) {                                                         \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), #x, __LINE__); \
      std::exit(1);                                                                 \
    }                                                                               \
  } while (0)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void read_kernel(const u32x4 *p, size_t n16, unsigned magic,
                                                   unsigned *sink) {
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= p[i];
  const unsigned v = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (v == magic) sink[0] = v;  // the host fills the buffers with 0x5a bytes: the fold is never magic
}

__global__ void empty_kernel() {}

static float graph_us(hipStream_t st, int calls, int reps,
                      const std::vector<std::function<void(hipStream_t)>> *fns, bool empty) {
  hipGraph_t g;
  hipGraphExec_t ge;
  CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
  for (int i = 0; i < calls; ++i) {
    if (empty)
      empty_kernel<<<1, 64, 0, st>>>();
    else
      (*fns)[i % fns->size()](st);
  }
  CK(hipStreamEndCapture(st, &g));
  CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
  CK(hipGraphLaunch(ge, st));
  CK(hipStreamSynchronize(st));
  hipEvent_t a, b;
  CK(hipEventCreate(&a));
  CK(hipEventCreate(&b));
  CK(hipEventRecord(a, st));
  for (int r = 0; r < reps; ++r) CK(hipGraphLaunch(ge, st));
  CK(hipEventRecord(b, st));
  CK(hipEventSynchronize(b));
  float ms = 0.f;
  CK(hipEventElapsedTime(&ms, a, b));
  CK(hipEventDestroy(a));
  CK(hipEventDestroy(b));
  CK(hipGraphExecDestroy(ge));
  CK(hipGraphDestroy(g));
  return ms * 1000.f / (float)(calls * reps);
}

int main(int argc, char **argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: %s BYTES [BYTES ...]\n", argv[0]);
    return 2;
  }
  hipStream_t st;
  CK(hipStreamCreate(&st));
  unsigned *sink;
  CK(hipMalloc(&sink, 64));
  for (int ai = 1; ai < argc; ++ai) {
    const size_t bytes = (std::strtoull(argv[ai], nullptr, 10) + 15) / 16 * 16;
    if (bytes == 0 || bytes > ((size_t)4 << 30)) {
      std::fprintf(stderr, "bytes out of range: %s\n", argv[ai]);
      return 2;
    }
    const size_t n16 = bytes / 16;
    const int copies = (int)std::max<size_t>(2, ((size_t)600 << 20) / bytes + 1);
    std::vector<void *> bufs(copies);
    for (auto &b : bufs) {
      CK(hipMalloc(&b, bytes));
      CK(hipMemset(b, 0x5a, bytes));
    }
    const size_t per_block = (size_t)256 * 4;  // 16-byte words per workgroup per iteration
    const unsigned blocks = (unsigned)std::max<size_t>(1, std::min<size_t>(2048, (n16 + per_block - 1) / per_block));
    std::vector<std::function<void(hipStream_t)>> fns;
    for (int c = 0; c < copies; ++c) {
      const u32x4 *p = static_cast<const u32x4 *>(bufs[c]);
      fns.push_back([=](hipStream_t s) { read_kernel<<<blocks, 256, 0, s>>>(p, n16, 0x9e3779b9u, sink); });
    }
    CK(hipDeviceSynchronize());
    std::vector<float> t;
    for (int r = 0; r < 7; ++r) t.push_back(graph_us(st, 20, 10, &fns, false));
    std::sort(t.begin(), t.end());
    const float med = t[t.size() / 2];
    std::printf("{\"bytes\": %zu, \"us\": %.3f, \"us_min\": %.3f, \"GBps\": %.1f, \"copies\": %d, \"blocks\": %u}\n",
                bytes, med, t[0], (double)bytes / med / 1e3, copies, blocks);
    std::fflush(stdout);
    for (auto &b : bufs) CK(hipFree(b));
  }
  std::vector<float> t;
  for (int r = 0; r < 5; ++r) t.push_back(graph_us(st, 64, 10, nullptr, true));
  std::sort(t.begin(), t.end());
  std::printf("{\"empty_launch_us\": %.3f}\n", t[t.size() / 2]);
  CK(hipFree(sink));
  return 0;
}
