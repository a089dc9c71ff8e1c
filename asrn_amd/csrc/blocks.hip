// Batched copies of small fp32 blocks in one launch: the layer's weight assembly (the concatenated and
// block-diagonal weights its fused GEMMs take, built from the parameters every step) and the scatter of their
// gradients back to the parameters. Each block is a rows x cols matrix copied from src (row stride sld) to dst (row
// stride dld), or filled with zeros when src is null; workgroups are numbered through the blocks in order.
#include "common.h"

namespace asrn {

constexpr int kCopyThreads = 256;
constexpr int kMaxBlocks = 16;

struct CopyBlock {
  const float* src; float* dst; int64_t sld, dld; int64_t rows, cols; int64_t first;   // first workgroup
};
struct CopyList {
  CopyBlock b[kMaxBlocks];
  int n;
};

__global__ __launch_bounds__(kCopyThreads) void k_copy_blocks(CopyList l) {
  int i = 0;
  while (i + 1 < l.n && (int64_t)blockIdx.x >= l.b[i + 1].first) ++i;
  const CopyBlock& c = l.b[i];
  const int64_t e = ((int64_t)blockIdx.x - c.first) * kCopyThreads + threadIdx.x;
  if (e >= c.rows * c.cols) return;
  const int64_t r = e / c.cols, k = e - r * c.cols;
  c.dst[r * c.dld + k] = c.src ? c.src[r * c.sld + k] : 0.f;
}

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_copy_blocks(int32_t n, const float* const* src, float* const* dst, const int64_t* sld,
                                const int64_t* dld, const int64_t* rows, const int64_t* cols, void* stream) {
  ASRN_REQUIRE(n >= 0 && n <= kMaxBlocks, "asrn_copy_blocks: %d blocks (at most %d per call)", n, kMaxBlocks);
  CopyList l = {};
  int64_t wg = 0;
  for (int i = 0; i < n; ++i) {
    ASRN_REQUIRE(rows[i] >= 0 && cols[i] >= 0 && dst[i] != nullptr && dld[i] >= cols[i] &&
                     (src[i] == nullptr || sld[i] >= cols[i]),
                 "asrn_copy_blocks: block %d: bad sizes (rows %lld, cols %lld, sld %lld, dld %lld) or null dst", i,
                 (long long)rows[i], (long long)cols[i], (long long)sld[i], (long long)dld[i]);
    l.b[i] = CopyBlock{src[i], dst[i], sld[i], dld[i], rows[i], cols[i], wg};
    wg += (rows[i] * cols[i] + kCopyThreads - 1) / kCopyThreads;
  }
  l.n = n;
  if (wg == 0) return 0;
  ASRN_REQUIRE(wg < (int64_t(1) << 31), "asrn_copy_blocks: too many elements");
  hipLaunchKernelGGL(k_copy_blocks, dim3((unsigned)wg), dim3(kCopyThreads), 0, (hipStream_t)stream, l);
  return check_launch("asrn_copy_blocks");
}
