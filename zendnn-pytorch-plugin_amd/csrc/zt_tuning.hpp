// Kernel-selection overrides of libzentorch_hip.so.
//
// Each knob is named after the environment variable that sets it.  The
// environment is read once, when the library is loaded; zt_set_tuning
// (include/zentorch_hip.h) changes a knob afterwards.  The host dispatch
// reads a knob with one atomic load, so no launch calls getenv and a change
// made while other threads launch is not a data race.
#pragma once

namespace zt {

enum Knob {
  kKnobWoqForceKernel,  // ZT_WOQ_FORCE_KERNEL: generic | decode | gemm | wide
  kKnobWoqDecodePlan,   // ZT_WOQ_DECODE_PLAN: "NK,NT,CPW,TPW" of the decode kernel
  kKnobWoqStream,       // ZT_WOQ_STREAM: "0" disables, "NW,CPW,TPW" forces a shape
  kKnobWoqWide,         // ZT_WOQ_WIDE: "0" disables, "KS" forces the K-split count
  kKnobWoqGemm,         // ZT_WOQ_GEMM: "o" 16x16 kernel, "d" 16x16 DMA, "1" 128x128, "w" / "v" / "x" load-wave kernel (4 / 3 stages, 256x192)
  kKnobWoqDebug,        // ZT_WOQ_DEBUG: print each launch shape to stderr
  kKnobWoqWave,         // ZT_WOQ_WAVE: "0" disables the wave-independent decode kernel
  kKnobWoqPersist,      // ZT_WOQ_PERSIST: "0" never, "1" / "2" force the persistent decode kernel (8 / 16 waves), "1p" / "2p" with gate_up tile pairs
  kKnobS8Skinny32,      // ZT_S8_SKINNY32: "TPW,PF,NW" of the 32-token skinny kernel
  kKnobS8Skinny,        // ZT_S8_SKINNY: "TPW,PF,NW" of the 16-token skinny kernel
  kKnobS8Frag,          // ZT_S8_FRAG: "0" never, "1" from M = 1 (fragment-order qx)
  kKnobS8Force,         // ZT_S8_FORCE: t tiled, s skinny, o 16x16 kernel
  kKnobS8Tile,          // ZT_S8_TILE: "2" 256 x 128 tiles, "9" 256 x 192, "1" 128 x 128, "0" 128 x 128 in 2 stages
  kKnobS8Kind,          // ZT_S8_KIND: w load-wave kernel (default), n 32x32 DMA kernel, r / 2 / 3 older kernels
  kKnobS8Split,         // ZT_S8_SPLIT: "0" disables the split-K skinny kernel, "2"-"4" its load depth
  kKnobMoeBn,           // ZT_MOE_BN: column tile of the MoE GEMMs
  kKnobWoqLean,         // ZT_WOQ_LEAN: "0" never, "1" forces the lean decode kernel wherever it applies, "p" too with gate_up tile pairs
  kKnobS8Fused,         // ZT_S8_FUSED: "0" never, "1" the quantise-in-prologue skinny kernel wherever it applies
  kKnobCount
};

// The knob's value, or nullptr when it is unset.
const char *knob(Knob k);

}  // namespace zt
