// O accumulator tiles of the 64-rows-per-wave attention kernels, held in
// AGPRs a[128:255] outside the compiler's register allocation: tile i is
// a[128 + 16 i : 143 + 16 i]. Every statement here names the registers it
// touches as clobbers, so the compiler keeps no value of its own in them
// across these statements; that it places none there at all is checked on
// the kernels' assembly by tests/test_agpr_reserve.py.
//
// Hazards (the compiler pads only the MFMAs it emits itself):
//  * an 8-pass XDL MFMA's result needs NumPasses + 3 wait states before a
//    VALU op reads or overwrites it: ot_pad() (24) precedes every read, scale
//    or zeroing that can follow the MFMAs;
//  * a VALU write of a register needs 2 wait states before an MFMA reads it:
//    ot_zero / ot_scale end with them, and the probabilities' producers are
//    separated from the MFMAs by mfma_src_fence().
#pragma once

#include "device_common.h"

namespace da {

#define DA_OT_CLOB_0 "a128","a129","a130","a131","a132","a133","a134","a135","a136","a137","a138","a139","a140","a141","a142","a143"
#define DA_OT_CLOB_1 "a144","a145","a146","a147","a148","a149","a150","a151","a152","a153","a154","a155","a156","a157","a158","a159"
#define DA_OT_CLOB_2 "a160","a161","a162","a163","a164","a165","a166","a167","a168","a169","a170","a171","a172","a173","a174","a175"
#define DA_OT_CLOB_3 "a176","a177","a178","a179","a180","a181","a182","a183","a184","a185","a186","a187","a188","a189","a190","a191"
#define DA_OT_CLOB_4 "a192","a193","a194","a195","a196","a197","a198","a199","a200","a201","a202","a203","a204","a205","a206","a207"
#define DA_OT_CLOB_5 "a208","a209","a210","a211","a212","a213","a214","a215","a216","a217","a218","a219","a220","a221","a222","a223"
#define DA_OT_CLOB_6 "a224","a225","a226","a227","a228","a229","a230","a231","a232","a233","a234","a235","a236","a237","a238","a239"
#define DA_OT_CLOB_7 "a240","a241","a242","a243","a244","a245","a246","a247","a248","a249","a250","a251","a252","a253","a254","a255"

__device__ __forceinline__ void ot_pad() { asm volatile("s_nop 15\n\ts_nop 7"); }

// a[tile I] += a b (32x32x16, bf16 or fp16 operands)
template <typename T, int I>
__device__ __forceinline__ void ot_mfma(u32x4 a, u32x4 b) {
  static_assert(I >= 0 && I < 8, "eight tiles");
  if constexpr (I == 0) {
    if constexpr (std::is_same<T, __bf16>::value)
      asm volatile("v_mfma_f32_32x32x16_bf16 a[128:143], %0, %1, a[128:143]" :: "v"(a), "v"(b) : DA_OT_CLOB_0);
    else
      asm volatile("v_mfma_f32_32x32x16_f16 a[128:143], %0, %1, a[128:143]" :: "v"(a), "v"(b) : DA_OT_CLOB_0);
  }
  if constexpr (I == 1) {
    if constexpr (std::is_same<T, __bf16>::value)
      asm volatile("v_mfma_f32_32x32x16_bf16 a[144:159], %0, %1, a[144:159]" :: "v"(a), "v"(b) : DA_OT_CLOB_1);
    else
      asm volatile("v_mfma_f32_32x32x16_f16 a[144:159], %0, %1, a[144:159]" :: "v"(a), "v"(b) : DA_OT_CLOB_1);
  }
  if constexpr (I == 2) {
    if constexpr (std::is_same<T, __bf16>::value)
      asm volatile("v_mfma_f32_32x32x16_bf16 a[160:175], %0, %1, a[160:175]" :: "v"(a), "v"(b) : DA_OT_CLOB_2);
    else
      asm volatile("v_mfma_f32_32x32x16_f16 a[160:175], %0, %1, a[160:175]" :: "v"(a), "v"(b) : DA_OT_CLOB_2);
  }
  if constexpr (I == 3) {
    if constexpr (std::is_same<T, __bf16>::value)
      asm volatile("v_mfma_f32_32x32x16_bf16 a[176:191], %0, %1, a[176:191]" :: "v"(a), "v"(b) : DA_OT_CLOB_3);
    else
      asm volatile("v_mfma_f32_32x32x16_f16 a[176:191], %0, %1, a[176:191]" :: "v"(a), "v"(b) : DA_OT_CLOB_3);
  }
  if constexpr (I == 4) {
    if constexpr (std::is_same<T, __bf16>::value)
      asm volatile("v_mfma_f32_32x32x16_bf16 a[192:207], %0, %1, a[192:207]" :: "v"(a), "v"(b) : DA_OT_CLOB_4);
    else
      asm volatile("v_mfma_f32_32x32x16_f16 a[192:207], %0, %1, a[192:207]" :: "v"(a), "v"(b) : DA_OT_CLOB_4);
  }
  if constexpr (I == 5) {
    if constexpr (std::is_same<T, __bf16>::value)
      asm volatile("v_mfma_f32_32x32x16_bf16 a[208:223], %0, %1, a[208:223]" :: "v"(a), "v"(b) : DA_OT_CLOB_5);
    else
      asm volatile("v_mfma_f32_32x32x16_f16 a[208:223], %0, %1, a[208:223]" :: "v"(a), "v"(b) : DA_OT_CLOB_5);
  }
  if constexpr (I == 6) {
    if constexpr (std::is_same<T, __bf16>::value)
      asm volatile("v_mfma_f32_32x32x16_bf16 a[224:239], %0, %1, a[224:239]" :: "v"(a), "v"(b) : DA_OT_CLOB_6);
    else
      asm volatile("v_mfma_f32_32x32x16_f16 a[224:239], %0, %1, a[224:239]" :: "v"(a), "v"(b) : DA_OT_CLOB_6);
  }
  if constexpr (I == 7) {
    if constexpr (std::is_same<T, __bf16>::value)
      asm volatile("v_mfma_f32_32x32x16_bf16 a[240:255], %0, %1, a[240:255]" :: "v"(a), "v"(b) : DA_OT_CLOB_7);
    else
      asm volatile("v_mfma_f32_32x32x16_f16 a[240:255], %0, %1, a[240:255]" :: "v"(a), "v"(b) : DA_OT_CLOB_7);
  }
}

// a[tile i] += a b for an index that is a constant after unrolling
template <typename T>
__device__ __forceinline__ void ot_mfma_at(int i, u32x4 a, u32x4 b) {
  switch (i) {
    case 0: ot_mfma<T, 0>(a, b); break;
    case 1: ot_mfma<T, 1>(a, b); break;
    case 2: ot_mfma<T, 2>(a, b); break;
    case 3: ot_mfma<T, 3>(a, b); break;
    case 4: ot_mfma<T, 4>(a, b); break;
    case 5: ot_mfma<T, 5>(a, b); break;
    case 6: ot_mfma<T, 6>(a, b); break;
    default: ot_mfma<T, 7>(a, b); break;
  }
}

// a[tile I] = 0
template <int I>
__device__ __forceinline__ void ot_zero() {
  if constexpr (I == 0) asm volatile("v_accvgpr_write_b32 a128, 0\n\tv_accvgpr_write_b32 a129, 0\n\tv_accvgpr_write_b32 a130, 0\n\tv_accvgpr_write_b32 a131, 0\n\tv_accvgpr_write_b32 a132, 0\n\tv_accvgpr_write_b32 a133, 0\n\tv_accvgpr_write_b32 a134, 0\n\tv_accvgpr_write_b32 a135, 0\n\tv_accvgpr_write_b32 a136, 0\n\tv_accvgpr_write_b32 a137, 0\n\tv_accvgpr_write_b32 a138, 0\n\tv_accvgpr_write_b32 a139, 0\n\tv_accvgpr_write_b32 a140, 0\n\tv_accvgpr_write_b32 a141, 0\n\tv_accvgpr_write_b32 a142, 0\n\tv_accvgpr_write_b32 a143, 0\n\ts_nop 1" ::: DA_OT_CLOB_0);
  if constexpr (I == 1) asm volatile("v_accvgpr_write_b32 a144, 0\n\tv_accvgpr_write_b32 a145, 0\n\tv_accvgpr_write_b32 a146, 0\n\tv_accvgpr_write_b32 a147, 0\n\tv_accvgpr_write_b32 a148, 0\n\tv_accvgpr_write_b32 a149, 0\n\tv_accvgpr_write_b32 a150, 0\n\tv_accvgpr_write_b32 a151, 0\n\tv_accvgpr_write_b32 a152, 0\n\tv_accvgpr_write_b32 a153, 0\n\tv_accvgpr_write_b32 a154, 0\n\tv_accvgpr_write_b32 a155, 0\n\tv_accvgpr_write_b32 a156, 0\n\tv_accvgpr_write_b32 a157, 0\n\tv_accvgpr_write_b32 a158, 0\n\tv_accvgpr_write_b32 a159, 0\n\ts_nop 1" ::: DA_OT_CLOB_1);
  if constexpr (I == 2) asm volatile("v_accvgpr_write_b32 a160, 0\n\tv_accvgpr_write_b32 a161, 0\n\tv_accvgpr_write_b32 a162, 0\n\tv_accvgpr_write_b32 a163, 0\n\tv_accvgpr_write_b32 a164, 0\n\tv_accvgpr_write_b32 a165, 0\n\tv_accvgpr_write_b32 a166, 0\n\tv_accvgpr_write_b32 a167, 0\n\tv_accvgpr_write_b32 a168, 0\n\tv_accvgpr_write_b32 a169, 0\n\tv_accvgpr_write_b32 a170, 0\n\tv_accvgpr_write_b32 a171, 0\n\tv_accvgpr_write_b32 a172, 0\n\tv_accvgpr_write_b32 a173, 0\n\tv_accvgpr_write_b32 a174, 0\n\tv_accvgpr_write_b32 a175, 0\n\ts_nop 1" ::: DA_OT_CLOB_2);
  if constexpr (I == 3) asm volatile("v_accvgpr_write_b32 a176, 0\n\tv_accvgpr_write_b32 a177, 0\n\tv_accvgpr_write_b32 a178, 0\n\tv_accvgpr_write_b32 a179, 0\n\tv_accvgpr_write_b32 a180, 0\n\tv_accvgpr_write_b32 a181, 0\n\tv_accvgpr_write_b32 a182, 0\n\tv_accvgpr_write_b32 a183, 0\n\tv_accvgpr_write_b32 a184, 0\n\tv_accvgpr_write_b32 a185, 0\n\tv_accvgpr_write_b32 a186, 0\n\tv_accvgpr_write_b32 a187, 0\n\tv_accvgpr_write_b32 a188, 0\n\tv_accvgpr_write_b32 a189, 0\n\tv_accvgpr_write_b32 a190, 0\n\tv_accvgpr_write_b32 a191, 0\n\ts_nop 1" ::: DA_OT_CLOB_3);
  if constexpr (I == 4) asm volatile("v_accvgpr_write_b32 a192, 0\n\tv_accvgpr_write_b32 a193, 0\n\tv_accvgpr_write_b32 a194, 0\n\tv_accvgpr_write_b32 a195, 0\n\tv_accvgpr_write_b32 a196, 0\n\tv_accvgpr_write_b32 a197, 0\n\tv_accvgpr_write_b32 a198, 0\n\tv_accvgpr_write_b32 a199, 0\n\tv_accvgpr_write_b32 a200, 0\n\tv_accvgpr_write_b32 a201, 0\n\tv_accvgpr_write_b32 a202, 0\n\tv_accvgpr_write_b32 a203, 0\n\tv_accvgpr_write_b32 a204, 0\n\tv_accvgpr_write_b32 a205, 0\n\tv_accvgpr_write_b32 a206, 0\n\tv_accvgpr_write_b32 a207, 0\n\ts_nop 1" ::: DA_OT_CLOB_4);
  if constexpr (I == 5) asm volatile("v_accvgpr_write_b32 a208, 0\n\tv_accvgpr_write_b32 a209, 0\n\tv_accvgpr_write_b32 a210, 0\n\tv_accvgpr_write_b32 a211, 0\n\tv_accvgpr_write_b32 a212, 0\n\tv_accvgpr_write_b32 a213, 0\n\tv_accvgpr_write_b32 a214, 0\n\tv_accvgpr_write_b32 a215, 0\n\tv_accvgpr_write_b32 a216, 0\n\tv_accvgpr_write_b32 a217, 0\n\tv_accvgpr_write_b32 a218, 0\n\tv_accvgpr_write_b32 a219, 0\n\tv_accvgpr_write_b32 a220, 0\n\tv_accvgpr_write_b32 a221, 0\n\tv_accvgpr_write_b32 a222, 0\n\tv_accvgpr_write_b32 a223, 0\n\ts_nop 1" ::: DA_OT_CLOB_5);
  if constexpr (I == 6) asm volatile("v_accvgpr_write_b32 a224, 0\n\tv_accvgpr_write_b32 a225, 0\n\tv_accvgpr_write_b32 a226, 0\n\tv_accvgpr_write_b32 a227, 0\n\tv_accvgpr_write_b32 a228, 0\n\tv_accvgpr_write_b32 a229, 0\n\tv_accvgpr_write_b32 a230, 0\n\tv_accvgpr_write_b32 a231, 0\n\tv_accvgpr_write_b32 a232, 0\n\tv_accvgpr_write_b32 a233, 0\n\tv_accvgpr_write_b32 a234, 0\n\tv_accvgpr_write_b32 a235, 0\n\tv_accvgpr_write_b32 a236, 0\n\tv_accvgpr_write_b32 a237, 0\n\tv_accvgpr_write_b32 a238, 0\n\tv_accvgpr_write_b32 a239, 0\n\ts_nop 1" ::: DA_OT_CLOB_6);
  if constexpr (I == 7) asm volatile("v_accvgpr_write_b32 a240, 0\n\tv_accvgpr_write_b32 a241, 0\n\tv_accvgpr_write_b32 a242, 0\n\tv_accvgpr_write_b32 a243, 0\n\tv_accvgpr_write_b32 a244, 0\n\tv_accvgpr_write_b32 a245, 0\n\tv_accvgpr_write_b32 a246, 0\n\tv_accvgpr_write_b32 a247, 0\n\tv_accvgpr_write_b32 a248, 0\n\tv_accvgpr_write_b32 a249, 0\n\tv_accvgpr_write_b32 a250, 0\n\tv_accvgpr_write_b32 a251, 0\n\tv_accvgpr_write_b32 a252, 0\n\tv_accvgpr_write_b32 a253, 0\n\tv_accvgpr_write_b32 a254, 0\n\tv_accvgpr_write_b32 a255, 0\n\ts_nop 1" ::: DA_OT_CLOB_7);
}

// a[tile I] *= s (per lane)
template <int I>
__device__ __forceinline__ void ot_scale(float s) {
  float t0, t1;
  if constexpr (I == 0)
    asm volatile("v_accvgpr_read_b32 %0, a128\n\tv_accvgpr_read_b32 %1, a129\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a128, %0\n\tv_accvgpr_write_b32 a129, %1\n\tv_accvgpr_read_b32 %0, a130\n\tv_accvgpr_read_b32 %1, a131\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a130, %0\n\tv_accvgpr_write_b32 a131, %1\n\tv_accvgpr_read_b32 %0, a132\n\tv_accvgpr_read_b32 %1, a133\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a132, %0\n\tv_accvgpr_write_b32 a133, %1\n\tv_accvgpr_read_b32 %0, a134\n\tv_accvgpr_read_b32 %1, a135\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a134, %0\n\tv_accvgpr_write_b32 a135, %1\n\tv_accvgpr_read_b32 %0, a136\n\tv_accvgpr_read_b32 %1, a137\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a136, %0\n\tv_accvgpr_write_b32 a137, %1\n\tv_accvgpr_read_b32 %0, a138\n\tv_accvgpr_read_b32 %1, a139\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a138, %0\n\tv_accvgpr_write_b32 a139, %1\n\tv_accvgpr_read_b32 %0, a140\n\tv_accvgpr_read_b32 %1, a141\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a140, %0\n\tv_accvgpr_write_b32 a141, %1\n\tv_accvgpr_read_b32 %0, a142\n\tv_accvgpr_read_b32 %1, a143\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a142, %0\n\tv_accvgpr_write_b32 a143, %1\n\ts_nop 1" : "=&v"(t0), "=&v"(t1) : "v"(s) : DA_OT_CLOB_0);
  if constexpr (I == 1)
    asm volatile("v_accvgpr_read_b32 %0, a144\n\tv_accvgpr_read_b32 %1, a145\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a144, %0\n\tv_accvgpr_write_b32 a145, %1\n\tv_accvgpr_read_b32 %0, a146\n\tv_accvgpr_read_b32 %1, a147\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a146, %0\n\tv_accvgpr_write_b32 a147, %1\n\tv_accvgpr_read_b32 %0, a148\n\tv_accvgpr_read_b32 %1, a149\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a148, %0\n\tv_accvgpr_write_b32 a149, %1\n\tv_accvgpr_read_b32 %0, a150\n\tv_accvgpr_read_b32 %1, a151\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a150, %0\n\tv_accvgpr_write_b32 a151, %1\n\tv_accvgpr_read_b32 %0, a152\n\tv_accvgpr_read_b32 %1, a153\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a152, %0\n\tv_accvgpr_write_b32 a153, %1\n\tv_accvgpr_read_b32 %0, a154\n\tv_accvgpr_read_b32 %1, a155\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a154, %0\n\tv_accvgpr_write_b32 a155, %1\n\tv_accvgpr_read_b32 %0, a156\n\tv_accvgpr_read_b32 %1, a157\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a156, %0\n\tv_accvgpr_write_b32 a157, %1\n\tv_accvgpr_read_b32 %0, a158\n\tv_accvgpr_read_b32 %1, a159\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a158, %0\n\tv_accvgpr_write_b32 a159, %1\n\ts_nop 1" : "=&v"(t0), "=&v"(t1) : "v"(s) : DA_OT_CLOB_1);
  if constexpr (I == 2)
    asm volatile("v_accvgpr_read_b32 %0, a160\n\tv_accvgpr_read_b32 %1, a161\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a160, %0\n\tv_accvgpr_write_b32 a161, %1\n\tv_accvgpr_read_b32 %0, a162\n\tv_accvgpr_read_b32 %1, a163\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a162, %0\n\tv_accvgpr_write_b32 a163, %1\n\tv_accvgpr_read_b32 %0, a164\n\tv_accvgpr_read_b32 %1, a165\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a164, %0\n\tv_accvgpr_write_b32 a165, %1\n\tv_accvgpr_read_b32 %0, a166\n\tv_accvgpr_read_b32 %1, a167\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a166, %0\n\tv_accvgpr_write_b32 a167, %1\n\tv_accvgpr_read_b32 %0, a168\n\tv_accvgpr_read_b32 %1, a169\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a168, %0\n\tv_accvgpr_write_b32 a169, %1\n\tv_accvgpr_read_b32 %0, a170\n\tv_accvgpr_read_b32 %1, a171\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a170, %0\n\tv_accvgpr_write_b32 a171, %1\n\tv_accvgpr_read_b32 %0, a172\n\tv_accvgpr_read_b32 %1, a173\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a172, %0\n\tv_accvgpr_write_b32 a173, %1\n\tv_accvgpr_read_b32 %0, a174\n\tv_accvgpr_read_b32 %1, a175\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a174, %0\n\tv_accvgpr_write_b32 a175, %1\n\ts_nop 1" : "=&v"(t0), "=&v"(t1) : "v"(s) : DA_OT_CLOB_2);
  if constexpr (I == 3)
    asm volatile("v_accvgpr_read_b32 %0, a176\n\tv_accvgpr_read_b32 %1, a177\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a176, %0\n\tv_accvgpr_write_b32 a177, %1\n\tv_accvgpr_read_b32 %0, a178\n\tv_accvgpr_read_b32 %1, a179\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a178, %0\n\tv_accvgpr_write_b32 a179, %1\n\tv_accvgpr_read_b32 %0, a180\n\tv_accvgpr_read_b32 %1, a181\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a180, %0\n\tv_accvgpr_write_b32 a181, %1\n\tv_accvgpr_read_b32 %0, a182\n\tv_accvgpr_read_b32 %1, a183\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a182, %0\n\tv_accvgpr_write_b32 a183, %1\n\tv_accvgpr_read_b32 %0, a184\n\tv_accvgpr_read_b32 %1, a185\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a184, %0\n\tv_accvgpr_write_b32 a185, %1\n\tv_accvgpr_read_b32 %0, a186\n\tv_accvgpr_read_b32 %1, a187\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a186, %0\n\tv_accvgpr_write_b32 a187, %1\n\tv_accvgpr_read_b32 %0, a188\n\tv_accvgpr_read_b32 %1, a189\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a188, %0\n\tv_accvgpr_write_b32 a189, %1\n\tv_accvgpr_read_b32 %0, a190\n\tv_accvgpr_read_b32 %1, a191\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a190, %0\n\tv_accvgpr_write_b32 a191, %1\n\ts_nop 1" : "=&v"(t0), "=&v"(t1) : "v"(s) : DA_OT_CLOB_3);
  if constexpr (I == 4)
    asm volatile("v_accvgpr_read_b32 %0, a192\n\tv_accvgpr_read_b32 %1, a193\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a192, %0\n\tv_accvgpr_write_b32 a193, %1\n\tv_accvgpr_read_b32 %0, a194\n\tv_accvgpr_read_b32 %1, a195\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a194, %0\n\tv_accvgpr_write_b32 a195, %1\n\tv_accvgpr_read_b32 %0, a196\n\tv_accvgpr_read_b32 %1, a197\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a196, %0\n\tv_accvgpr_write_b32 a197, %1\n\tv_accvgpr_read_b32 %0, a198\n\tv_accvgpr_read_b32 %1, a199\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a198, %0\n\tv_accvgpr_write_b32 a199, %1\n\tv_accvgpr_read_b32 %0, a200\n\tv_accvgpr_read_b32 %1, a201\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a200, %0\n\tv_accvgpr_write_b32 a201, %1\n\tv_accvgpr_read_b32 %0, a202\n\tv_accvgpr_read_b32 %1, a203\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a202, %0\n\tv_accvgpr_write_b32 a203, %1\n\tv_accvgpr_read_b32 %0, a204\n\tv_accvgpr_read_b32 %1, a205\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a204, %0\n\tv_accvgpr_write_b32 a205, %1\n\tv_accvgpr_read_b32 %0, a206\n\tv_accvgpr_read_b32 %1, a207\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a206, %0\n\tv_accvgpr_write_b32 a207, %1\n\ts_nop 1" : "=&v"(t0), "=&v"(t1) : "v"(s) : DA_OT_CLOB_4);
  if constexpr (I == 5)
    asm volatile("v_accvgpr_read_b32 %0, a208\n\tv_accvgpr_read_b32 %1, a209\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a208, %0\n\tv_accvgpr_write_b32 a209, %1\n\tv_accvgpr_read_b32 %0, a210\n\tv_accvgpr_read_b32 %1, a211\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a210, %0\n\tv_accvgpr_write_b32 a211, %1\n\tv_accvgpr_read_b32 %0, a212\n\tv_accvgpr_read_b32 %1, a213\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a212, %0\n\tv_accvgpr_write_b32 a213, %1\n\tv_accvgpr_read_b32 %0, a214\n\tv_accvgpr_read_b32 %1, a215\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a214, %0\n\tv_accvgpr_write_b32 a215, %1\n\tv_accvgpr_read_b32 %0, a216\n\tv_accvgpr_read_b32 %1, a217\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a216, %0\n\tv_accvgpr_write_b32 a217, %1\n\tv_accvgpr_read_b32 %0, a218\n\tv_accvgpr_read_b32 %1, a219\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a218, %0\n\tv_accvgpr_write_b32 a219, %1\n\tv_accvgpr_read_b32 %0, a220\n\tv_accvgpr_read_b32 %1, a221\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a220, %0\n\tv_accvgpr_write_b32 a221, %1\n\tv_accvgpr_read_b32 %0, a222\n\tv_accvgpr_read_b32 %1, a223\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a222, %0\n\tv_accvgpr_write_b32 a223, %1\n\ts_nop 1" : "=&v"(t0), "=&v"(t1) : "v"(s) : DA_OT_CLOB_5);
  if constexpr (I == 6)
    asm volatile("v_accvgpr_read_b32 %0, a224\n\tv_accvgpr_read_b32 %1, a225\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a224, %0\n\tv_accvgpr_write_b32 a225, %1\n\tv_accvgpr_read_b32 %0, a226\n\tv_accvgpr_read_b32 %1, a227\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a226, %0\n\tv_accvgpr_write_b32 a227, %1\n\tv_accvgpr_read_b32 %0, a228\n\tv_accvgpr_read_b32 %1, a229\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a228, %0\n\tv_accvgpr_write_b32 a229, %1\n\tv_accvgpr_read_b32 %0, a230\n\tv_accvgpr_read_b32 %1, a231\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a230, %0\n\tv_accvgpr_write_b32 a231, %1\n\tv_accvgpr_read_b32 %0, a232\n\tv_accvgpr_read_b32 %1, a233\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a232, %0\n\tv_accvgpr_write_b32 a233, %1\n\tv_accvgpr_read_b32 %0, a234\n\tv_accvgpr_read_b32 %1, a235\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a234, %0\n\tv_accvgpr_write_b32 a235, %1\n\tv_accvgpr_read_b32 %0, a236\n\tv_accvgpr_read_b32 %1, a237\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a236, %0\n\tv_accvgpr_write_b32 a237, %1\n\tv_accvgpr_read_b32 %0, a238\n\tv_accvgpr_read_b32 %1, a239\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a238, %0\n\tv_accvgpr_write_b32 a239, %1\n\ts_nop 1" : "=&v"(t0), "=&v"(t1) : "v"(s) : DA_OT_CLOB_6);
  if constexpr (I == 7)
    asm volatile("v_accvgpr_read_b32 %0, a240\n\tv_accvgpr_read_b32 %1, a241\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a240, %0\n\tv_accvgpr_write_b32 a241, %1\n\tv_accvgpr_read_b32 %0, a242\n\tv_accvgpr_read_b32 %1, a243\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a242, %0\n\tv_accvgpr_write_b32 a243, %1\n\tv_accvgpr_read_b32 %0, a244\n\tv_accvgpr_read_b32 %1, a245\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a244, %0\n\tv_accvgpr_write_b32 a245, %1\n\tv_accvgpr_read_b32 %0, a246\n\tv_accvgpr_read_b32 %1, a247\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a246, %0\n\tv_accvgpr_write_b32 a247, %1\n\tv_accvgpr_read_b32 %0, a248\n\tv_accvgpr_read_b32 %1, a249\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a248, %0\n\tv_accvgpr_write_b32 a249, %1\n\tv_accvgpr_read_b32 %0, a250\n\tv_accvgpr_read_b32 %1, a251\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a250, %0\n\tv_accvgpr_write_b32 a251, %1\n\tv_accvgpr_read_b32 %0, a252\n\tv_accvgpr_read_b32 %1, a253\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a252, %0\n\tv_accvgpr_write_b32 a253, %1\n\tv_accvgpr_read_b32 %0, a254\n\tv_accvgpr_read_b32 %1, a255\n\tv_mul_f32 %0, %2, %0\n\tv_mul_f32 %1, %2, %1\n\tv_accvgpr_write_b32 a254, %0\n\tv_accvgpr_write_b32 a255, %1\n\ts_nop 1" : "=&v"(t0), "=&v"(t1) : "v"(s) : DA_OT_CLOB_7);
}

// the 16 accumulator elements of tile I
template <int I>
__device__ __forceinline__ f32x16 ot_read() {
  float x[16];
  if constexpr (I == 0) asm volatile("v_accvgpr_read_b32 %0, a128\n\tv_accvgpr_read_b32 %1, a129\n\tv_accvgpr_read_b32 %2, a130\n\tv_accvgpr_read_b32 %3, a131\n\tv_accvgpr_read_b32 %4, a132\n\tv_accvgpr_read_b32 %5, a133\n\tv_accvgpr_read_b32 %6, a134\n\tv_accvgpr_read_b32 %7, a135\n\tv_accvgpr_read_b32 %8, a136\n\tv_accvgpr_read_b32 %9, a137\n\tv_accvgpr_read_b32 %10, a138\n\tv_accvgpr_read_b32 %11, a139\n\tv_accvgpr_read_b32 %12, a140\n\tv_accvgpr_read_b32 %13, a141\n\tv_accvgpr_read_b32 %14, a142\n\tv_accvgpr_read_b32 %15, a143" : "=v"(x[0]), "=v"(x[1]), "=v"(x[2]), "=v"(x[3]), "=v"(x[4]), "=v"(x[5]), "=v"(x[6]), "=v"(x[7]), "=v"(x[8]), "=v"(x[9]), "=v"(x[10]), "=v"(x[11]), "=v"(x[12]), "=v"(x[13]), "=v"(x[14]), "=v"(x[15]) :: DA_OT_CLOB_0);
  if constexpr (I == 1) asm volatile("v_accvgpr_read_b32 %0, a144\n\tv_accvgpr_read_b32 %1, a145\n\tv_accvgpr_read_b32 %2, a146\n\tv_accvgpr_read_b32 %3, a147\n\tv_accvgpr_read_b32 %4, a148\n\tv_accvgpr_read_b32 %5, a149\n\tv_accvgpr_read_b32 %6, a150\n\tv_accvgpr_read_b32 %7, a151\n\tv_accvgpr_read_b32 %8, a152\n\tv_accvgpr_read_b32 %9, a153\n\tv_accvgpr_read_b32 %10, a154\n\tv_accvgpr_read_b32 %11, a155\n\tv_accvgpr_read_b32 %12, a156\n\tv_accvgpr_read_b32 %13, a157\n\tv_accvgpr_read_b32 %14, a158\n\tv_accvgpr_read_b32 %15, a159" : "=v"(x[0]), "=v"(x[1]), "=v"(x[2]), "=v"(x[3]), "=v"(x[4]), "=v"(x[5]), "=v"(x[6]), "=v"(x[7]), "=v"(x[8]), "=v"(x[9]), "=v"(x[10]), "=v"(x[11]), "=v"(x[12]), "=v"(x[13]), "=v"(x[14]), "=v"(x[15]) :: DA_OT_CLOB_1);
  if constexpr (I == 2) asm volatile("v_accvgpr_read_b32 %0, a160\n\tv_accvgpr_read_b32 %1, a161\n\tv_accvgpr_read_b32 %2, a162\n\tv_accvgpr_read_b32 %3, a163\n\tv_accvgpr_read_b32 %4, a164\n\tv_accvgpr_read_b32 %5, a165\n\tv_accvgpr_read_b32 %6, a166\n\tv_accvgpr_read_b32 %7, a167\n\tv_accvgpr_read_b32 %8, a168\n\tv_accvgpr_read_b32 %9, a169\n\tv_accvgpr_read_b32 %10, a170\n\tv_accvgpr_read_b32 %11, a171\n\tv_accvgpr_read_b32 %12, a172\n\tv_accvgpr_read_b32 %13, a173\n\tv_accvgpr_read_b32 %14, a174\n\tv_accvgpr_read_b32 %15, a175" : "=v"(x[0]), "=v"(x[1]), "=v"(x[2]), "=v"(x[3]), "=v"(x[4]), "=v"(x[5]), "=v"(x[6]), "=v"(x[7]), "=v"(x[8]), "=v"(x[9]), "=v"(x[10]), "=v"(x[11]), "=v"(x[12]), "=v"(x[13]), "=v"(x[14]), "=v"(x[15]) :: DA_OT_CLOB_2);
  if constexpr (I == 3) asm volatile("v_accvgpr_read_b32 %0, a176\n\tv_accvgpr_read_b32 %1, a177\n\tv_accvgpr_read_b32 %2, a178\n\tv_accvgpr_read_b32 %3, a179\n\tv_accvgpr_read_b32 %4, a180\n\tv_accvgpr_read_b32 %5, a181\n\tv_accvgpr_read_b32 %6, a182\n\tv_accvgpr_read_b32 %7, a183\n\tv_accvgpr_read_b32 %8, a184\n\tv_accvgpr_read_b32 %9, a185\n\tv_accvgpr_read_b32 %10, a186\n\tv_accvgpr_read_b32 %11, a187\n\tv_accvgpr_read_b32 %12, a188\n\tv_accvgpr_read_b32 %13, a189\n\tv_accvgpr_read_b32 %14, a190\n\tv_accvgpr_read_b32 %15, a191" : "=v"(x[0]), "=v"(x[1]), "=v"(x[2]), "=v"(x[3]), "=v"(x[4]), "=v"(x[5]), "=v"(x[6]), "=v"(x[7]), "=v"(x[8]), "=v"(x[9]), "=v"(x[10]), "=v"(x[11]), "=v"(x[12]), "=v"(x[13]), "=v"(x[14]), "=v"(x[15]) :: DA_OT_CLOB_3);
  if constexpr (I == 4) asm volatile("v_accvgpr_read_b32 %0, a192\n\tv_accvgpr_read_b32 %1, a193\n\tv_accvgpr_read_b32 %2, a194\n\tv_accvgpr_read_b32 %3, a195\n\tv_accvgpr_read_b32 %4, a196\n\tv_accvgpr_read_b32 %5, a197\n\tv_accvgpr_read_b32 %6, a198\n\tv_accvgpr_read_b32 %7, a199\n\tv_accvgpr_read_b32 %8, a200\n\tv_accvgpr_read_b32 %9, a201\n\tv_accvgpr_read_b32 %10, a202\n\tv_accvgpr_read_b32 %11, a203\n\tv_accvgpr_read_b32 %12, a204\n\tv_accvgpr_read_b32 %13, a205\n\tv_accvgpr_read_b32 %14, a206\n\tv_accvgpr_read_b32 %15, a207" : "=v"(x[0]), "=v"(x[1]), "=v"(x[2]), "=v"(x[3]), "=v"(x[4]), "=v"(x[5]), "=v"(x[6]), "=v"(x[7]), "=v"(x[8]), "=v"(x[9]), "=v"(x[10]), "=v"(x[11]), "=v"(x[12]), "=v"(x[13]), "=v"(x[14]), "=v"(x[15]) :: DA_OT_CLOB_4);
  if constexpr (I == 5) asm volatile("v_accvgpr_read_b32 %0, a208\n\tv_accvgpr_read_b32 %1, a209\n\tv_accvgpr_read_b32 %2, a210\n\tv_accvgpr_read_b32 %3, a211\n\tv_accvgpr_read_b32 %4, a212\n\tv_accvgpr_read_b32 %5, a213\n\tv_accvgpr_read_b32 %6, a214\n\tv_accvgpr_read_b32 %7, a215\n\tv_accvgpr_read_b32 %8, a216\n\tv_accvgpr_read_b32 %9, a217\n\tv_accvgpr_read_b32 %10, a218\n\tv_accvgpr_read_b32 %11, a219\n\tv_accvgpr_read_b32 %12, a220\n\tv_accvgpr_read_b32 %13, a221\n\tv_accvgpr_read_b32 %14, a222\n\tv_accvgpr_read_b32 %15, a223" : "=v"(x[0]), "=v"(x[1]), "=v"(x[2]), "=v"(x[3]), "=v"(x[4]), "=v"(x[5]), "=v"(x[6]), "=v"(x[7]), "=v"(x[8]), "=v"(x[9]), "=v"(x[10]), "=v"(x[11]), "=v"(x[12]), "=v"(x[13]), "=v"(x[14]), "=v"(x[15]) :: DA_OT_CLOB_5);
  if constexpr (I == 6) asm volatile("v_accvgpr_read_b32 %0, a224\n\tv_accvgpr_read_b32 %1, a225\n\tv_accvgpr_read_b32 %2, a226\n\tv_accvgpr_read_b32 %3, a227\n\tv_accvgpr_read_b32 %4, a228\n\tv_accvgpr_read_b32 %5, a229\n\tv_accvgpr_read_b32 %6, a230\n\tv_accvgpr_read_b32 %7, a231\n\tv_accvgpr_read_b32 %8, a232\n\tv_accvgpr_read_b32 %9, a233\n\tv_accvgpr_read_b32 %10, a234\n\tv_accvgpr_read_b32 %11, a235\n\tv_accvgpr_read_b32 %12, a236\n\tv_accvgpr_read_b32 %13, a237\n\tv_accvgpr_read_b32 %14, a238\n\tv_accvgpr_read_b32 %15, a239" : "=v"(x[0]), "=v"(x[1]), "=v"(x[2]), "=v"(x[3]), "=v"(x[4]), "=v"(x[5]), "=v"(x[6]), "=v"(x[7]), "=v"(x[8]), "=v"(x[9]), "=v"(x[10]), "=v"(x[11]), "=v"(x[12]), "=v"(x[13]), "=v"(x[14]), "=v"(x[15]) :: DA_OT_CLOB_6);
  if constexpr (I == 7) asm volatile("v_accvgpr_read_b32 %0, a240\n\tv_accvgpr_read_b32 %1, a241\n\tv_accvgpr_read_b32 %2, a242\n\tv_accvgpr_read_b32 %3, a243\n\tv_accvgpr_read_b32 %4, a244\n\tv_accvgpr_read_b32 %5, a245\n\tv_accvgpr_read_b32 %6, a246\n\tv_accvgpr_read_b32 %7, a247\n\tv_accvgpr_read_b32 %8, a248\n\tv_accvgpr_read_b32 %9, a249\n\tv_accvgpr_read_b32 %10, a250\n\tv_accvgpr_read_b32 %11, a251\n\tv_accvgpr_read_b32 %12, a252\n\tv_accvgpr_read_b32 %13, a253\n\tv_accvgpr_read_b32 %14, a254\n\tv_accvgpr_read_b32 %15, a255" : "=v"(x[0]), "=v"(x[1]), "=v"(x[2]), "=v"(x[3]), "=v"(x[4]), "=v"(x[5]), "=v"(x[6]), "=v"(x[7]), "=v"(x[8]), "=v"(x[9]), "=v"(x[10]), "=v"(x[11]), "=v"(x[12]), "=v"(x[13]), "=v"(x[14]), "=v"(x[15]) :: DA_OT_CLOB_7);
  f32x16 r;
#pragma unroll
  for (int j = 0; j < 16; ++j) r[j] = x[j];
  return r;
}

}  // namespace da
