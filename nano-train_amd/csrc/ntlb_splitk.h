// Split-K tail shared by the 256x256-tile GEMMs (512 threads, 8 waves of
// 128x64, fp32 accumulators acc[8][4] of 16x16 blocks per lane).
//
// A dense tiling runs one workgroup per tile, one per compute unit.  When the
// tiles past the last whole wave (rem = tiles mod CUs) would fill at most half
// the chip, each of them is cut into s K ranges run by s workgroups at the end
// of the grid.  Each range writes its fp32 partial tile to a caller workspace;
// the last range to arrive sums all s partials in range order (the same order
// every call, so results do not depend on arrival order) and runs the normal
// epilogue.  Nobody waits on another workgroup.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

namespace ntlb {

constexpr int SPLIT_THREADS = 512;
constexpr int SPLIT_PART4 = SPLIT_THREADS * 32;  // float4 per partial tile (128 fp32 per thread)

struct SplitPlan {
  int base, s, tail;
};

inline int split_device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cus[dev] = c;
  }
  return cus[dev];
}

// The plan for `tiles` output tiles of nk K blocks: split_s = 1 means no
// split.  Each range keeps at least min_blocks K blocks: shorter ranges lose
// more to the partial tiles' round trip than they gain.
inline SplitPlan split_plan(int64_t tiles, int nk, int min_blocks) {
  SplitPlan p{(int)tiles, 1, 0};
  const int64_t cus = split_device_cus();
  const int64_t full = (tiles / cus) * cus, rem = tiles - full;
  if (rem == 0 || rem * 2 > cus) return p;
  int s = (int)std::min<int64_t>(cus / rem, 8);
  s = std::min(s, nk / min_blocks);
  if (s < 2) return p;
  p.base = (int)full;
  p.s = s;
  p.tail = (int)rem;
  return p;
}

// Workspace layout: the tile counters, then the fp32 partials
// [tail][s][SPLIT_PART4 float4].  The counter area is the same for every plan
// on a device (one uint32 per possible tail tile: a plan's tail is at most
// half the compute units), so calls of different shapes on one workspace find
// their counters where the previous call left them, at zero.
inline int64_t split_count_bytes() { return ((int64_t)split_device_cus() / 2 * 4 + 255) / 256 * 256; }

inline int64_t split_ws_bytes(const SplitPlan& p) {
  if (p.s < 2) return 0;
  return split_count_bytes() + (int64_t)p.tail * p.s * SPLIT_PART4 * 16;
}

// Which tile and K range workgroup pid takes: pid < base keeps its tile and
// all K blocks (chunk -1); the others take chunk (q % s) of tile base + q / s.
struct SplitWork {
  int pid;    // the output tile
  int tail;   // tail tile index, or -1
  int chunk;  // K range index within the tile
};

// Workgroup pid runs on XCD pid % 8.  When base % 8 == 0, tail unit q runs
// on XCD q % 8 too, and q is renumbered so that each XCD walks a contiguous
// range of tail units: the chunks of one tail tile and the tiles next to it in
// the raster then share that XCD's L2 (c3 dgrad: 2278 -> 2316 TFLOP/s).  The
// renumbering only moves units between workgroups: every tile's chunks, and
// the order they are summed in, stay the same.
__device__ __forceinline__ SplitWork split_work(int pid, int base, int s) {
  SplitWork w{pid, -1, 0};
  if (s > 1 && pid >= base) {
    int q = pid - base;
    if ((base & 7) == 0) {
      const int n = (int)gridDim.x - base;
      const int xcd = q & 7, local = q >> 3;
      const int per = n >> 3, extra = n & 7;
      q = xcd * per + min(xcd, extra) + local;
    }
    w.tail = q / s;
    w.chunk = q - w.tail * s;
    w.pid = base + w.tail;
  }
  return w;
}

// acc = sum over chunks c = 0..s-1, in that order, of the partial tiles at
// part + c * SPLIT_PART4 (float4 units, this thread's slot 0):
// ((p0 + p1) + p2) + ...  Rounds of 16 loads (four slots of four chunks)
// are in flight at once; one instance serves every s.
template <typename V4>
__device__ __forceinline__ void split_sum_partials(V4 (&acc)[8][4], const float4* part, int s) {
  for (int c0 = 0; c0 < s; c0 += 4) {
#pragma unroll
    for (int r = 0; r < 32; r += 4) {
      float4 v[4][4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int cc = min(c0 + c, s - 1);  // in bounds; chunks past s are not added
#pragma unroll
        for (int k = 0; k < 4; ++k) v[c][k] = part[(int64_t)cc * SPLIT_PART4 + (r + k) * SPLIT_THREADS];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        V4& a = acc[(r + k) >> 2][(r + k) & 3];
        V4 t = (V4){v[0][k].x, v[0][k].y, v[0][k].z, v[0][k].w};
        if (c0 > 0) t = a + t;
#pragma unroll
        for (int c = 1; c < 4; ++c)
          if (c0 + c < s) t += (V4){v[c][k].x, v[c][k].y, v[c][k].z, v[c][k].w};
        a = t;
      }
    }
  }
}

// Publish this range's partial tile; returns true in the last range to
// arrive, whose acc then holds the sum of all ranges (and which resets the
// tile's counter for the next call), false in the others, which are done.
// Stores are lane-major: every store instruction writes 1 KiB of consecutive
// memory.  Every thread of the workgroup must call it.
template <typename V4>
__device__ __forceinline__ bool split_exchange(V4 (&acc)[8][4], float* ws, uint32_t* ws_count, int tail, int s,
                                               int chunk, int tid) {
  float4* part = reinterpret_cast<float4*>(ws) + (int64_t)tail * s * SPLIT_PART4 + tid;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      part[(int64_t)chunk * SPLIT_PART4 + (i * 4 + j) * SPLIT_THREADS] =
          make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
  // every wave's stores are complete in this XCD's L2 after the barrier; one
  // agent-scope release then writes them back before the count
  __syncthreads();
  __shared__ int split_last;
  if (tid == 0)
    split_last = __hip_atomic_fetch_add(ws_count + tail, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) ==
                 (uint32_t)(s - 1);
  __syncthreads();
  if (!split_last) return false;
  if (tid == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  __syncthreads();
  split_sum_partials(acc, part, s);
  if (tid == 0) atomicExch(ws_count + tail, 0u);  // ready for the next call
  return true;
}

}  // namespace ntlb
