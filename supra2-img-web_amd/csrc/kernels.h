// Internal interface between the C ABI (api.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sa {

// Everything a kernel needs for one attention call, resolved and validated by the host.
constexpr int kMaxOrder = 256;  // sequences a launch schedule can order (kernel-argument bytes)

struct AttnParams {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  int64_t q_off, k_off, v_off, o_off;
  int64_t ldq, ldk, ldv, ldo;
  int64_t sq, sk, sv, so;
  int B, H, D, Lq, Lk;
  float scale_log2;  // softmax scale * log2(e): scores are kept in the base-2 domain
  int bias_mode;
  const float* bias;
  int64_t sbias;
  const int32_t* lut;
  int num_buckets;
  int mask_mode;
  const int32_t* key_len;
  const uint8_t* key_mask;
  int64_t smask;
  // Host copy of key_len (or null): the input of the sequence schedule, which the host makes once
  // the kernel is chosen. Never read by a kernel.
  const int32_t* key_len_host;
  // Sequence schedule of the flash kernel: sequence rank r (its position in the launch order)
  // runs sequence order[r] when order_n > 0, sequence r otherwise. Kernel-argument data, so the
  // lookup is a scalar load and needs no device allocation.
  int order_n;
  uint8_t order[kMaxOrder];
};

enum { BIAS_NONE = 0, BIAS_DENSE = 1, BIAS_RELPOS = 2 };
enum { MASK_NONE = 0, MASK_KEY_LEN = 1, MASK_KEY_MASK = 2 };
// Variant only (never an ABI value): key lengths plus a launch shaped by their host copy. Flash
// kernel: the sequence schedule in AttnParams::order, so that the plain key-length variant does not
// read the schedule at all. 16-query small-launch kernel: sequences packed by their key blocks.
constexpr int MASK_KEY_LEN_ORDERED = 3;

// Arguments of the flash kernels, packed into 112 bytes: the runtime starts launches with at most
// 112 bytes of explicit arguments about 0.8 us sooner than larger ones (measured back to back on
// MI355X), a tenth of a small call. Pointers carry the callers' element offsets; strides are 32-bit
// (calls with larger strides take the generic kernel).
struct FlashArgs {
  const float* q;  // q + q_off (likewise k, v, o)
  const float* k;
  const float* v;
  float* o;
  int32_t sq, sk, sv, so;      // batch strides
  int32_t ldq, ldk, ldv, ldo;  // row strides
  int32_t Lq, Lk;
  int32_t tiles;               // workgroups of the launch (the grid size, for the XCD remap)
  int16_t H, num_buckets;
  float scale_log2;
  int32_t aux;       // start-up stagger period in workgroups (unbiased single-split kernels) | key-mask row stride
  const void* mask;  // key lengths (int32) | key mask (uint8)
  const float* bias; // dense bias | relative-position table
  union {
    const int32_t* lut;  // relative-position bucket LUT
    int64_t sbias;       // dense bias batch stride
    struct {
      int32_t first, count;  // folded launch: the 64-query units [first, first + count) left over
    } fold;
  };
};
static_assert(sizeof(FlashArgs) == 112, "flash kernel arguments must stay within 112 bytes");
// The packed arguments of a call whose launch has `tiles` workgroups (flash_mfma_args_fit(p)).
FlashArgs flash_args(const AttnParams& p, int64_t tiles);

// Flash kernel on fp32 MFMA for D in {64, 128} with 16-byte aligned rows.
// nsplit in {1, 2}: key blocks are split across the 4 waves of a workgroup (small head-dim-64
// launches take flash_small instead). num_cus (the device's CU count) sets the start-up stagger of
// the single-split kernels.
hipError_t launch_flash_mfma(const AttnParams& p, int nsplit, int num_cus, hipStream_t stream);
const char* flash_mfma_name(int D, int nsplit);
// The flash kernels take 32-bit strides, at most 32767 heads and buckets; other calls take the
// generic kernel.
bool flash_mfma_args_fit(const AttnParams& p);

// One compiled flash_mfma_kernel instantiation: <D, nsplit, bias (BIAS_*), mask (MASK_* or
// MASK_KEY_LEN_ORDERED)>.
struct FlashVariant {
  int D, nsplit, bias, mask;
};
// The variant a call launches with this key split.
FlashVariant flash_mfma_variant(const AttnParams& p, int nsplit);
// Workgroups of that launch.
int64_t flash_mfma_workgroups(const AttnParams& p, int nsplit, int num_cus);
// Queries per workgroup of the flash kernel with this key split, and the workgroups of that variant
// one CU holds at once (4 for the unbiased head-dim-64 single-split kernels, 1 for the others).
int flash_mfma_unit_queries(int nsplit);
int flash_mfma_per_cu(const AttnParams& p, int nsplit);
// Units (128-query tiles) of a flash launch that go to a second launch (0 = none), the kernel of
// that launch, and the work items [*first, *first + count) it runs (returns count): 32-query groups
// of flash_small, or 64-query units of the 2-way key-split flash kernel.
constexpr int TAIL_NONE = 0, TAIL_SMALL = 1, TAIL_SPLIT2 = 2, TAIL_FOLD = 3;
int64_t flash_mfma_tail_units(const AttnParams& p, int nsplit, int num_cus);
int flash_mfma_tail_kernel(const AttnParams& p, int nsplit, int num_cus);
int64_t flash_mfma_tail_groups(const AttnParams& p, int nsplit, int num_cus, int64_t* first);
// 32-query groups [first, first + count) of the call through flash_small_kernel (no key mask).
hipError_t launch_flash_small_groups(const AttnParams& p, int64_t first, int64_t count, hipStream_t stream);
// Every compiled variant, in a fixed order: returns the count and fills out[0, min(count, cap)).
int flash_mfma_variants(FlashVariant* out, int cap);

// Small launches with head dim 64 (csrc/flash_small.hip): one workgroup per group of 32 queries,
// its key blocks dealt to 4 waves with K and V in registers; variants <64, 4, bias, mask> with mask
// in {MASK_NONE, MASK_KEY_LEN, MASK_KEY_MASK} (no sequence schedule).
int flash_small_waves(const AttnParams& p);
int64_t flash_small_workgroups(const AttnParams& p);
const char* flash_small_name(int nw);
int flash_small_variants(FlashVariant* out, int cap);
hipError_t launch_flash_small(const AttnParams& p, hipStream_t stream);

// Launches of at most this many workgroups run one per CU on MI355X (the small-launch kernels).
constexpr int kSmallLaunchCUs = 256;

// Small launches with head dim 64 in groups of 16 queries (csrc/flash_small16.hip): one workgroup of
// 4 waves per 16 queries of one (sequence, head), v_mfma_f32_16x16x4f32; variants <bias, mask> with
// mask in {MASK_NONE, MASK_KEY_LEN, MASK_KEY_MASK, MASK_KEY_LEN_ORDERED}. The last packs sequences
// of at most two key blocks (host key lengths, B <= 16) at 2 or 1 waves per 16-query group, so
// their workgroups hold 2 or 4 groups, where that makes a launch of more than kSmallLaunchCUs
// workgroups fit.
int64_t flash_small16_workgroups(const AttnParams& p);
FlashVariant flash_small16_variant(const AttnParams& p);
const char* flash_small16_name();
int flash_small16_variants(FlashVariant* out, int cap);
hipError_t launch_flash_small16(const AttnParams& p, hipStream_t stream);

// Wide heads (D = 256 or 512; no bias or a dense one; no mask, key lengths or a key mask): head dim
// split across the waves of a workgroup (D = 256) or score blocks dealt to them (D = 512), keys
// split across workgroups, partials merged by a second kernel via a workspace.
constexpr int kWideMaxChunks = 16;
// Largest merge-record workspace a plan may ask for: the allocation-free entry point's per-GPU
// scratch, so that entry point takes every wide-head call the workspace entry point takes.
constexpr int64_t kWideMaxRecordBytes = int64_t(32) << 20;
struct WidePlan {
  int q_groups;       // 32-query groups per (sequence, head)
  int nks;            // key chunks per split group (workgroups sharing one query group; 1: none split)
  int chunk;          // keys per chunk of a split group (multiple of 32)
  int whole_chunk;    // keys of an unsplit group's one chunk (all of them, in whole rounds of the kernel)
  int64_t whole;      // with nks > 1: leading groups, in (sequence, head, group) order, that run
                      // unsplit in a launch of their own before the split ones (0: every group split)
  int64_t ws_floats;  // workspace floats (0 when nks == 1)
};
bool wide_mfma_supported(const AttnParams& p);
// Every compiled variant <D, 1, bias, mask>, in a fixed order (as flash_mfma_variants).
int wide_mfma_variants(FlashVariant* out, int cap);
WidePlan wide_mfma_plan(const AttnParams& p, int num_cus);
const char* wide_mfma_name(int D);
hipError_t launch_wide_mfma(const AttnParams& p, const WidePlan& plan, float* ws, hipStream_t stream);

// Any head dim up to 1024, any alignment: one workgroup per query row.
hipError_t launch_generic(const AttnParams& p, hipStream_t stream);

// Dense [H, Lq, Lk] relative-position bias from a table and bucket LUT.
hipError_t launch_position_bias(const float* table, const int32_t* lut, int num_buckets, int H, int Lq,
                                int Lk, float* out, hipStream_t stream);

constexpr int GENERIC_MAX_D = 1024;

// ---- linear layer y = epilogue(alpha * x W^T) (csrc/linear_mfma.hip)
enum { LIN_ACT_NONE = 0, LIN_ACT_GELU = 1, LIN_ACT_GELU_TANH = 2, LIN_ACT_SILU = 3 };
enum { LIN_EPI_STORE = 0, LIN_EPI_RESID = 1, LIN_EPI_RESID_GATE = 2 };
struct LinearParams {
  const float* x;  // [M, K] rows at x + x_off + m*ldx
  int64_t x_off, ldx;
  const float* w;  // [N, K] rows at w + n*ldw
  int64_t ldw;
  const float* bias;  // [N] or null
  const float* gate;  // gate[gate_off + n] (LIN_EPI_RESID_GATE)
  int64_t gate_off;
  float* y;  // [M, N] rows at y + y_off + m*ldy
  int64_t y_off, ldy;
  // residual epilogues: the added rows are read from resid (same offset and stride as y) instead
  // of y itself when non-null, so y = r + resid needs no copy of resid into y first
  const float* resid;
  int M, N, K;
  float alpha;
  int act, epi;
};
struct LinearTile {
  int wm, wn;  // 32x32 accumulators per wave along M and N (tile 64*wm x 64*wn)
  int bk, ns;  // k-tile depth and LDS stages
  int ksplit;  // k splits of linear_ksplit_kernel (4: 32 x 32 tiles, 2: 32 x 64 tiles), 0: linear_mfma_kernel
};
// MFMA kernel when K % 8 == 0 and x, W rows are 16-byte aligned; the generic kernel otherwise.
bool linear_mfma_supported(const LinearParams& p);
LinearTile linear_mfma_tile(const LinearParams& p, int num_cus);
const char* linear_kernel_name(const LinearParams& p, int num_cus);
hipError_t launch_linear(const LinearParams& p, int num_cus, hipStream_t stream);

// ---- GroupNorm over an NHWC image [HW, C] in `groups` channel groups (csrc/groupnorm.hip).
// part: scratch of 3 * groups * groupnorm_chunks(HW, groups) floats for the chunk statistics.
int groupnorm_chunks(int HW, int groups);
hipError_t launch_groupnorm(const float* x, const float* gamma, const float* beta, float* y, float* part, int HW, int C,
                            int groups, float eps, hipStream_t stream);

}  // namespace sa
