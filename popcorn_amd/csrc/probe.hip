// Matrix-core rate probe: one wave per SIMD on every CU runs back-to-back
// bf16 32x32x16 products (v_mfma_f32_32x32x16_bf16) on random operands that
// change from product to product, optionally with the attention forward's
// per-score vector work beside each product (an fma, an exponential, a sum and
// half a packing). Each wave reports the shader-clock cycles (s_memtime) and
// the 100 MHz real-time ticks (s_memrealtime) its loop took, so the caller gets
// the products' issue rate per cycle and the clock the chip ran them at.
//
// The measured figure is the bf16 matrix rate this board sustains under its
// power limit with operands that toggle like real data; it bounds every
// matrix-bound kernel here from above (the published 2.5 PFLOP/s assumes the
// 2.4 GHz peak clock). No counterpart in Popcorn: a measurement aid for the
// bench, not an operator.
//
// The streaming probe is the HBM counterpart: the fastest stream form found
// for these kernels (one 16-byte non-temporal vector per thread, 64-thread
// blocks, one vector per thread in all) copying one input or combining two,
// which gives the ceiling that a streaming kernel with the same reads and
// writes per byte can reach at a given size.
//
// Registers of the matrix-core probe are named in the assembly: fragments in v200-v231, the vector
// work in v232-v238, accumulators in a0-a127, all declared clobbered, so the
// compiler keeps nothing of its own there. Nothing is read from memory; the
// only store is the per-wave timing pair.

#include "api.h"
#include "common.h"

namespace pk {
namespace {

constexpr int kProbeThreads = 256;  // one wave per SIMD of a CU

template <bool SOFTMAX>
__global__ __attribute__((amdgpu_flat_work_group_size(kProbeThreads, kProbeThreads), amdgpu_waves_per_eu(1, 1)))
void mfma_probe_kernel(uint64_t* out, int iters) {
  // bf16 pairs in [0.5, 2) with random signs and mantissas, different per lane and per fragment
  uint32_t x = (blockIdx.x * kProbeThreads + threadIdx.x) * 2654435761u + 12345u;
  uint32_t w[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    w[j] = (x & 0x807f807fu) | 0x3f003f00u;
  }
  asm volatile(
      "v_mov_b32 v200, %0\n"
      "v_mov_b32 v201, %1\n"
      "v_mov_b32 v202, %2\n"
      "v_mov_b32 v203, %3\n"
      "v_mov_b32 v204, %4\n"
      "v_mov_b32 v205, %5\n"
      "v_mov_b32 v206, %6\n"
      "v_mov_b32 v207, %7\n"
      "v_mov_b32 v208, %8\n"
      "v_mov_b32 v209, %9\n"
      "v_mov_b32 v210, %10\n"
      "v_mov_b32 v211, %11\n"
      "v_mov_b32 v212, %12\n"
      "v_mov_b32 v213, %13\n"
      "v_mov_b32 v214, %14\n"
      "v_mov_b32 v215, %15\n"
      "v_mov_b32 v216, %16\n"
      "v_mov_b32 v217, %17\n"
      "v_mov_b32 v218, %18\n"
      "v_mov_b32 v219, %19\n"
      "v_mov_b32 v220, %20\n"
      "v_mov_b32 v221, %21\n"
      "v_mov_b32 v222, %22\n"
      "v_mov_b32 v223, %23\n"
      "v_mov_b32 v224, %24\n"
      "v_mov_b32 v225, %25\n"
      "v_mov_b32 v226, %26\n"
      "v_mov_b32 v227, %27\n"
      "v_mov_b32 v228, %28\n"
      "v_mov_b32 v229, %29\n"
      "v_mov_b32 v230, %30\n"
      "v_mov_b32 v231, %31\n"
      "s_mov_b32 s0, 0x3f000000\n"
      "v_mov_b32 v232, 0\n"
      "v_mov_b32 v233, 0\n"
      "v_mov_b32 v234, 0\n"
      "v_mov_b32 v235, 0\n"
      "v_mov_b32 v236, 0\n"
      "v_mov_b32 v237, 0\n"
      "v_accvgpr_write_b32 a0, 0\n"
      "v_accvgpr_write_b32 a1, 0\n"
      "v_accvgpr_write_b32 a2, 0\n"
      "v_accvgpr_write_b32 a3, 0\n"
      "v_accvgpr_write_b32 a4, 0\n"
      "v_accvgpr_write_b32 a5, 0\n"
      "v_accvgpr_write_b32 a6, 0\n"
      "v_accvgpr_write_b32 a7, 0\n"
      "v_accvgpr_write_b32 a8, 0\n"
      "v_accvgpr_write_b32 a9, 0\n"
      "v_accvgpr_write_b32 a10, 0\n"
      "v_accvgpr_write_b32 a11, 0\n"
      "v_accvgpr_write_b32 a12, 0\n"
      "v_accvgpr_write_b32 a13, 0\n"
      "v_accvgpr_write_b32 a14, 0\n"
      "v_accvgpr_write_b32 a15, 0\n"
      "v_accvgpr_write_b32 a16, 0\n"
      "v_accvgpr_write_b32 a17, 0\n"
      "v_accvgpr_write_b32 a18, 0\n"
      "v_accvgpr_write_b32 a19, 0\n"
      "v_accvgpr_write_b32 a20, 0\n"
      "v_accvgpr_write_b32 a21, 0\n"
      "v_accvgpr_write_b32 a22, 0\n"
      "v_accvgpr_write_b32 a23, 0\n"
      "v_accvgpr_write_b32 a24, 0\n"
      "v_accvgpr_write_b32 a25, 0\n"
      "v_accvgpr_write_b32 a26, 0\n"
      "v_accvgpr_write_b32 a27, 0\n"
      "v_accvgpr_write_b32 a28, 0\n"
      "v_accvgpr_write_b32 a29, 0\n"
      "v_accvgpr_write_b32 a30, 0\n"
      "v_accvgpr_write_b32 a31, 0\n"
      "v_accvgpr_write_b32 a32, 0\n"
      "v_accvgpr_write_b32 a33, 0\n"
      "v_accvgpr_write_b32 a34, 0\n"
      "v_accvgpr_write_b32 a35, 0\n"
      "v_accvgpr_write_b32 a36, 0\n"
      "v_accvgpr_write_b32 a37, 0\n"
      "v_accvgpr_write_b32 a38, 0\n"
      "v_accvgpr_write_b32 a39, 0\n"
      "v_accvgpr_write_b32 a40, 0\n"
      "v_accvgpr_write_b32 a41, 0\n"
      "v_accvgpr_write_b32 a42, 0\n"
      "v_accvgpr_write_b32 a43, 0\n"
      "v_accvgpr_write_b32 a44, 0\n"
      "v_accvgpr_write_b32 a45, 0\n"
      "v_accvgpr_write_b32 a46, 0\n"
      "v_accvgpr_write_b32 a47, 0\n"
      "v_accvgpr_write_b32 a48, 0\n"
      "v_accvgpr_write_b32 a49, 0\n"
      "v_accvgpr_write_b32 a50, 0\n"
      "v_accvgpr_write_b32 a51, 0\n"
      "v_accvgpr_write_b32 a52, 0\n"
      "v_accvgpr_write_b32 a53, 0\n"
      "v_accvgpr_write_b32 a54, 0\n"
      "v_accvgpr_write_b32 a55, 0\n"
      "v_accvgpr_write_b32 a56, 0\n"
      "v_accvgpr_write_b32 a57, 0\n"
      "v_accvgpr_write_b32 a58, 0\n"
      "v_accvgpr_write_b32 a59, 0\n"
      "v_accvgpr_write_b32 a60, 0\n"
      "v_accvgpr_write_b32 a61, 0\n"
      "v_accvgpr_write_b32 a62, 0\n"
      "v_accvgpr_write_b32 a63, 0\n"
      "v_accvgpr_write_b32 a64, 0\n"
      "v_accvgpr_write_b32 a65, 0\n"
      "v_accvgpr_write_b32 a66, 0\n"
      "v_accvgpr_write_b32 a67, 0\n"
      "v_accvgpr_write_b32 a68, 0\n"
      "v_accvgpr_write_b32 a69, 0\n"
      "v_accvgpr_write_b32 a70, 0\n"
      "v_accvgpr_write_b32 a71, 0\n"
      "v_accvgpr_write_b32 a72, 0\n"
      "v_accvgpr_write_b32 a73, 0\n"
      "v_accvgpr_write_b32 a74, 0\n"
      "v_accvgpr_write_b32 a75, 0\n"
      "v_accvgpr_write_b32 a76, 0\n"
      "v_accvgpr_write_b32 a77, 0\n"
      "v_accvgpr_write_b32 a78, 0\n"
      "v_accvgpr_write_b32 a79, 0\n"
      "v_accvgpr_write_b32 a80, 0\n"
      "v_accvgpr_write_b32 a81, 0\n"
      "v_accvgpr_write_b32 a82, 0\n"
      "v_accvgpr_write_b32 a83, 0\n"
      "v_accvgpr_write_b32 a84, 0\n"
      "v_accvgpr_write_b32 a85, 0\n"
      "v_accvgpr_write_b32 a86, 0\n"
      "v_accvgpr_write_b32 a87, 0\n"
      "v_accvgpr_write_b32 a88, 0\n"
      "v_accvgpr_write_b32 a89, 0\n"
      "v_accvgpr_write_b32 a90, 0\n"
      "v_accvgpr_write_b32 a91, 0\n"
      "v_accvgpr_write_b32 a92, 0\n"
      "v_accvgpr_write_b32 a93, 0\n"
      "v_accvgpr_write_b32 a94, 0\n"
      "v_accvgpr_write_b32 a95, 0\n"
      "v_accvgpr_write_b32 a96, 0\n"
      "v_accvgpr_write_b32 a97, 0\n"
      "v_accvgpr_write_b32 a98, 0\n"
      "v_accvgpr_write_b32 a99, 0\n"
      "v_accvgpr_write_b32 a100, 0\n"
      "v_accvgpr_write_b32 a101, 0\n"
      "v_accvgpr_write_b32 a102, 0\n"
      "v_accvgpr_write_b32 a103, 0\n"
      "v_accvgpr_write_b32 a104, 0\n"
      "v_accvgpr_write_b32 a105, 0\n"
      "v_accvgpr_write_b32 a106, 0\n"
      "v_accvgpr_write_b32 a107, 0\n"
      "v_accvgpr_write_b32 a108, 0\n"
      "v_accvgpr_write_b32 a109, 0\n"
      "v_accvgpr_write_b32 a110, 0\n"
      "v_accvgpr_write_b32 a111, 0\n"
      "v_accvgpr_write_b32 a112, 0\n"
      "v_accvgpr_write_b32 a113, 0\n"
      "v_accvgpr_write_b32 a114, 0\n"
      "v_accvgpr_write_b32 a115, 0\n"
      "v_accvgpr_write_b32 a116, 0\n"
      "v_accvgpr_write_b32 a117, 0\n"
      "v_accvgpr_write_b32 a118, 0\n"
      "v_accvgpr_write_b32 a119, 0\n"
      "v_accvgpr_write_b32 a120, 0\n"
      "v_accvgpr_write_b32 a121, 0\n"
      "v_accvgpr_write_b32 a122, 0\n"
      "v_accvgpr_write_b32 a123, 0\n"
      "v_accvgpr_write_b32 a124, 0\n"
      "v_accvgpr_write_b32 a125, 0\n"
      "v_accvgpr_write_b32 a126, 0\n"
      "v_accvgpr_write_b32 a127, 0\n"
      :: "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]), "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]), "v"(w[16]), "v"(w[17]), "v"(w[18]), "v"(w[19]), "v"(w[20]), "v"(w[21]), "v"(w[22]), "v"(w[23]), "v"(w[24]), "v"(w[25]), "v"(w[26]), "v"(w[27]), "v"(w[28]), "v"(w[29]), "v"(w[30]), "v"(w[31])
      : "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207", "v208", "v209", "v210", "v211", "v212", "v213", "v214", "v215", "v216", "v217", "v218", "v219", "v220", "v221", "v222", "v223", "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234", "v235", "v236", "v237", "v238", "v239", "a0", "a1", "a2", "a3", "a4", "a5", "a6", "a7", "a8", "a9", "a10", "a11", "a12", "a13", "a14", "a15", "a16", "a17", "a18", "a19", "a20", "a21", "a22", "a23", "a24", "a25", "a26", "a27", "a28", "a29", "a30", "a31", "a32", "a33", "a34", "a35", "a36", "a37", "a38", "a39", "a40", "a41", "a42", "a43", "a44", "a45", "a46", "a47", "a48", "a49", "a50", "a51", "a52", "a53", "a54", "a55", "a56", "a57", "a58", "a59", "a60", "a61", "a62", "a63", "a64", "a65", "a66", "a67", "a68", "a69", "a70", "a71", "a72", "a73", "a74", "a75", "a76", "a77", "a78", "a79", "a80", "a81", "a82", "a83", "a84", "a85", "a86", "a87", "a88", "a89", "a90", "a91", "a92", "a93", "a94", "a95", "a96", "a97", "a98", "a99", "a100", "a101", "a102", "a103", "a104", "a105", "a106", "a107", "a108", "a109", "a110", "a111", "a112", "a113", "a114", "a115", "a116", "a117", "a118", "a119", "a120", "a121", "a122", "a123", "a124", "a125", "a126", "a127", "s0");
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
    if constexpr (SOFTMAX)
      asm volatile(
          "v_mfma_f32_32x32x16_bf16 a[0:15], v[200:203], v[212:215], a[0:15]\n"
          "v_fma_f32 v232, v232, s0, -v236\n"
          "v_exp_f32 v232, v232\n"
          "s_nop 0\n"
          "v_add_f32 v237, v237, v232\n"
          "v_mfma_f32_32x32x16_bf16 a[16:31], v[204:207], v[216:219], a[16:31]\n"
          "v_fma_f32 v233, v233, s0, -v236\n"
          "v_exp_f32 v233, v233\n"
          "s_nop 0\n"
          "v_add_f32 v237, v237, v233\n"
          "v_cvt_pk_bf16_f32 v238, v233, v237\n"
          "v_mfma_f32_32x32x16_bf16 a[32:47], v[208:211], v[220:223], a[32:47]\n"
          "v_fma_f32 v234, v234, s0, -v236\n"
          "v_exp_f32 v234, v234\n"
          "s_nop 0\n"
          "v_add_f32 v237, v237, v234\n"
          "v_mfma_f32_32x32x16_bf16 a[48:63], v[212:215], v[224:227], a[48:63]\n"
          "v_fma_f32 v235, v235, s0, -v236\n"
          "v_exp_f32 v235, v235\n"
          "s_nop 0\n"
          "v_add_f32 v237, v237, v235\n"
          "v_cvt_pk_bf16_f32 v238, v235, v237\n"
          "v_mfma_f32_32x32x16_bf16 a[64:79], v[216:219], v[228:231], a[64:79]\n"
          "v_fma_f32 v232, v232, s0, -v236\n"
          "v_exp_f32 v232, v232\n"
          "s_nop 0\n"
          "v_add_f32 v237, v237, v232\n"
          "v_mfma_f32_32x32x16_bf16 a[80:95], v[220:223], v[200:203], a[80:95]\n"
          "v_fma_f32 v233, v233, s0, -v236\n"
          "v_exp_f32 v233, v233\n"
          "s_nop 0\n"
          "v_add_f32 v237, v237, v233\n"
          "v_cvt_pk_bf16_f32 v238, v233, v237\n"
          "v_mfma_f32_32x32x16_bf16 a[96:111], v[224:227], v[204:207], a[96:111]\n"
          "v_fma_f32 v234, v234, s0, -v236\n"
          "v_exp_f32 v234, v234\n"
          "s_nop 0\n"
          "v_add_f32 v237, v237, v234\n"
          "v_mfma_f32_32x32x16_bf16 a[112:127], v[228:231], v[208:211], a[112:127]\n"
          "v_fma_f32 v235, v235, s0, -v236\n"
          "v_exp_f32 v235, v235\n"
          "s_nop 0\n"
          "v_add_f32 v237, v237, v235\n"
          "v_cvt_pk_bf16_f32 v238, v235, v237\n"
          ::: "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207", "v208", "v209", "v210", "v211", "v212", "v213", "v214", "v215", "v216", "v217", "v218", "v219", "v220", "v221", "v222", "v223", "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234", "v235", "v236", "v237", "v238", "v239", "a0", "a1", "a2", "a3", "a4", "a5", "a6", "a7", "a8", "a9", "a10", "a11", "a12", "a13", "a14", "a15", "a16", "a17", "a18", "a19", "a20", "a21", "a22", "a23", "a24", "a25", "a26", "a27", "a28", "a29", "a30", "a31", "a32", "a33", "a34", "a35", "a36", "a37", "a38", "a39", "a40", "a41", "a42", "a43", "a44", "a45", "a46", "a47", "a48", "a49", "a50", "a51", "a52", "a53", "a54", "a55", "a56", "a57", "a58", "a59", "a60", "a61", "a62", "a63", "a64", "a65", "a66", "a67", "a68", "a69", "a70", "a71", "a72", "a73", "a74", "a75", "a76", "a77", "a78", "a79", "a80", "a81", "a82", "a83", "a84", "a85", "a86", "a87", "a88", "a89", "a90", "a91", "a92", "a93", "a94", "a95", "a96", "a97", "a98", "a99", "a100", "a101", "a102", "a103", "a104", "a105", "a106", "a107", "a108", "a109", "a110", "a111", "a112", "a113", "a114", "a115", "a116", "a117", "a118", "a119", "a120", "a121", "a122", "a123", "a124", "a125", "a126", "a127");
    else
      asm volatile(
          "v_mfma_f32_32x32x16_bf16 a[0:15], v[200:203], v[212:215], a[0:15]\n"
          "v_mfma_f32_32x32x16_bf16 a[16:31], v[204:207], v[216:219], a[16:31]\n"
          "v_mfma_f32_32x32x16_bf16 a[32:47], v[208:211], v[220:223], a[32:47]\n"
          "v_mfma_f32_32x32x16_bf16 a[48:63], v[212:215], v[224:227], a[48:63]\n"
          "v_mfma_f32_32x32x16_bf16 a[64:79], v[216:219], v[228:231], a[64:79]\n"
          "v_mfma_f32_32x32x16_bf16 a[80:95], v[220:223], v[200:203], a[80:95]\n"
          "v_mfma_f32_32x32x16_bf16 a[96:111], v[224:227], v[204:207], a[96:111]\n"
          "v_mfma_f32_32x32x16_bf16 a[112:127], v[228:231], v[208:211], a[112:127]\n"
          ::: "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207", "v208", "v209", "v210", "v211", "v212", "v213", "v214", "v215", "v216", "v217", "v218", "v219", "v220", "v221", "v222", "v223", "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234", "v235", "v236", "v237", "v238", "v239", "a0", "a1", "a2", "a3", "a4", "a5", "a6", "a7", "a8", "a9", "a10", "a11", "a12", "a13", "a14", "a15", "a16", "a17", "a18", "a19", "a20", "a21", "a22", "a23", "a24", "a25", "a26", "a27", "a28", "a29", "a30", "a31", "a32", "a33", "a34", "a35", "a36", "a37", "a38", "a39", "a40", "a41", "a42", "a43", "a44", "a45", "a46", "a47", "a48", "a49", "a50", "a51", "a52", "a53", "a54", "a55", "a56", "a57", "a58", "a59", "a60", "a61", "a62", "a63", "a64", "a65", "a66", "a67", "a68", "a69", "a70", "a71", "a72", "a73", "a74", "a75", "a76", "a77", "a78", "a79", "a80", "a81", "a82", "a83", "a84", "a85", "a86", "a87", "a88", "a89", "a90", "a91", "a92", "a93", "a94", "a95", "a96", "a97", "a98", "a99", "a100", "a101", "a102", "a103", "a104", "a105", "a106", "a107", "a108", "a109", "a110", "a111", "a112", "a113", "a114", "a115", "a116", "a117", "a118", "a119", "a120", "a121", "a122", "a123", "a124", "a125", "a126", "a127");
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");  // the last products retire
  const uint64_t c1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x % 64 == 0) {
    const int wave = blockIdx.x * (kProbeThreads / 64) + threadIdx.x / 64;
    out[2 * wave] = c1 - c0;
    out[2 * wave + 1] = r1 - r0;
  }
}

constexpr int kStreamThreads = 64;

// y = a (one read) or y = a ^ b (two reads), one 16-byte vector per thread
template <bool TWO>
__global__ __launch_bounds__(kStreamThreads) void stream_probe_kernel(const u32x4* a, const u32x4* b, u32x4* y,
                                                                      int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kStreamThreads + threadIdx.x;
  if (i >= n) return;
  u32x4 v = __builtin_nontemporal_load(a + i);
  if constexpr (TWO) v ^= __builtin_nontemporal_load(b + i);
  __builtin_nontemporal_store(v, y + i);
}

}  // namespace
}  // namespace pk

extern "C" {

int pk_probe_stream(const void* a, const void* b, void* y, int64_t bytes, int reads, void* stream) {
  using namespace pk;
  if (reads != 1 && reads != 2) return fail(PK_ERR_INVALID, "pk_probe_stream: reads %d is neither 1 nor 2", reads);
  if (bytes < 0 || bytes % 16) return fail(PK_ERR_INVALID, "pk_probe_stream: %lld bytes is not a multiple of 16",
                                            (long long)bytes);
  if (bytes == 0) return PK_OK;
  if (!a || !y || (reads == 2 && !b)) return fail(PK_ERR_INVALID, "pk_probe_stream: null pointer");
  if (!aligned16(a) || !aligned16(y) || (reads == 2 && !aligned16(b)))
    return fail(PK_ERR_INVALID, "pk_probe_stream: pointers must be 16-byte aligned");
  const int64_t n = bytes / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((n + kStreamThreads - 1) / kStreamThreads));
  if (reads == 2)
    hipLaunchKernelGGL(stream_probe_kernel<true>, grid, dim3(kStreamThreads), 0, s, static_cast<const u32x4*>(a),
                       static_cast<const u32x4*>(b), static_cast<u32x4*>(y), n);
  else
    hipLaunchKernelGGL(stream_probe_kernel<false>, grid, dim3(kStreamThreads), 0, s, static_cast<const u32x4*>(a),
                       nullptr, static_cast<u32x4*>(y), n);
  return launched("pk_probe_stream");
}

int pk_probe_mfma(int softmax, int iters, int blocks, uint64_t* out, void* stream) {
  using namespace pk;
  if (iters < 1 || blocks < 1)
    return fail(PK_ERR_INVALID, "pk_probe_mfma: iters %d and blocks %d must be positive", iters, blocks);
  if (!out) return fail(PK_ERR_INVALID, "pk_probe_mfma: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (softmax)
    hipLaunchKernelGGL(mfma_probe_kernel<true>, dim3(blocks), dim3(kProbeThreads), 0, s, out, iters);
  else
    hipLaunchKernelGGL(mfma_probe_kernel<false>, dim3(blocks), dim3(kProbeThreads), 0, s, out, iters);
  return launched("pk_probe_mfma");
}

}  // extern "C"
