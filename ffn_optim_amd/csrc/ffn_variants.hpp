// ffn_variants.hpp -- the macro-tile variants compiled into libffn_mi355x.so.
//
// X(id, BM, BN, BK, waves along M, waves along N, LDS stages[, sync slot, DMA k-steps (of 16 K),
//   waves along K, waves issuing the refill, refill-only waves, early refill loads, MFMA block
//   edge (32: 32x32x16, 16: 16x16x32)])
// (DMA k-steps covering the whole stage spread a deep pipeline's refill over the whole
// iteration.)  The K-sliced 128x128 tiles (10, 11) give each wave a 128x64 wave tile
// over half of every stage: a quarter fewer fragment reads per MFMA than 64x64 wave tiles,
// for the down GEMMs whose output has about one 128x128 tile per CU.  Variant 13 runs it with
// eight waves (2x2 along M and N, 64x64 wave tiles), two per SIMD, so one wave's MFMAs cover
// the other's LDS and barrier waits.  Variant 12 runs the
// 256x256 tile with eight waves (two per SIMD, 128x64 wave tiles): when every CU holds a
// single tile, the second wave of a SIMD issues MFMAs while the first waits on LDS or DMA.
// Its refill goes out in the first k-step of the iteration (2% faster on the DiT-size up),
// issued by waves 0-3 alone, one per SIMD (2-4% faster on the DiT-size GEMMs than all
// eight waves sharing it), and half of it earlier still: 8 of each refilling wave's 16 loads go
// out in the slots after the previous iteration's stage barrier, when the stage they fill is
// free (last argument; DiT-size up and Stream-K down 1.4% and 2-3% faster on whole steps).
// Variants 17-21 are variants 1, 13, 16, 15 and 11 with more waves that only refill the LDS
// stages (four; two for the two-wave 15): each SIMD holds refill waves beside tile waves that
// never wait on the texture unit.  DiT-size Basic down -1.6% (17), its 1536-deep shard -8%;
// unaligned up -4% (18) and Basic down -8.5% (19); aligned mid-size Basic down -3 to -6% (21,
// whose 128x64 wave tiles read less LDS per MFMA than variant 13's 64x64, with two waves per
// SIMD now); decode Basic down -18% (20) while its weights stay in
// the last-level cache (smoke and decode-shard FFNs; the full decode FFN streams them from HBM
// at the same rate either way).
// Variants 22-25 take 16x16x32 MFMAs.  Under the DiT-size FFN's load the clock is held
// down by the chip's activity, and a 16x16x32 MFMA takes about 10% less energy per FLOP than a
// 32x32x16 one (register-only MFMA streams at 1.35 kW: 675 against 750 J per PFLOP), so the
// same power buys a higher clock (up GEMM 1826 against 1663 MHz).  Variant 22 is variant 12's
// 256x256 tile with 64x128 wave tiles (4x2 waves: 12 fragments of 16 rows per k-step instead of
// 16 for 128x64), its stage barrier at slot 23 of 32 and three quarters of each refill issued
// early, the rest in the first quarter of the iteration: at the higher clock the down GEMM's
// operands need the longer lead (DiT-size, one interleaved run against variant 12: up 472.5 ->
// 448.5 us, Stream-K down 464.1 -> 445.9 us, whole FFN 953.6 -> 918.2 us).  Variant 23 is
// variant 17 with 16x16x32 blocks, variant 24 variant 21 (the K-sliced 128x128 tile, its slices
// exchanging 16x16 blocks): aligned mid-size Basic down 31.8 -> 29.7 us (the 16x16 forms of
// variants 18 and 19 gained 1% on the unaligned FFN, within the noise: not kept).  Variant 25
// is a 256x192 tile of 16x16 blocks (64x96 wave tiles, barrier at slot 17 of 24, 10 of 14
// refill loads early) for the DiT FFN's H/8 shard, whose up GEMM has 192 tiles of 256x256 on 256
// CUs and 256 of 256x192: shard up 74.5 -> 62.6 us, Basic FFN 137.4 -> 128.5 us.
// The deep-pipeline 64-row tiles (8, 9) keep 56 KiB or more of weights in flight per CU for
// the memory-bound small-M (decode) shapes.  Variant 14 K-slices the 64x64 tile (64x32 wave
// tiles over half of every stage): two MFMAs per k-step per wave instead of one, for the
// latency-bound down GEMMs with one 64x64 tile per CU (-8 to -9% on the unaligned mid-size
// and the decode Basic down).
// Each variant is built for both storage types in its own object, with every launch role:
// the up epilogues (GELU-erf, GELU-rational, SiLU, and SwiGLU where its wave tiles hold whole
// 64-column block pairs), the plain store of the down GEMM, the Stream-K form of the store and
// of the GELU / SiLU up (split tiles finished in the launch), and gathered-row forms of the up
// roles for an X read in place as a strided view.
#pragma once

#define FFN_VARIANTS(X)                     \
    X(0, 256, 256, 64, 2, 2, 2, 9)          \
    X(1, 256, 128, 64, 2, 2, 3, -1, 4)      \
    X(2, 128, 256, 64, 2, 2, 3)             \
    X(3, 128, 128, 64, 2, 2, 2)             \
    X(4, 64, 64, 64, 2, 2, 2)               \
    X(5, 64, 128, 64, 2, 2, 3)              \
    X(6, 256, 256, 32, 2, 2, 4, -1, 2)      \
    X(7, 256, 256, 32, 2, 2, 5, -1, 2)      \
    X(8, 64, 64, 64, 2, 2, 8, -1, 4)        \
    X(9, 64, 128, 64, 2, 2, 6)              \
    X(10, 128, 128, 64, 1, 2, 5, -1, 2, 2)  \
    X(11, 128, 128, 64, 1, 2, 4, -1, 2, 2)  \
    X(12, 256, 256, 64, 2, 4, 2, -1, 1, 1, 4, 0, 8) \
    X(13, 128, 128, 64, 2, 2, 4, 3, 2, 2)   \
    X(14, 64, 64, 64, 1, 2, 6, -1, 2, 2)    \
    X(15, 32, 32, 128, 1, 1, 8, -1, 4, 2)   \
    X(16, 64, 64, 128, 1, 2, 5, -1, 4, 2)   \
    X(17, 256, 128, 64, 2, 2, 3, -1, 4, 1, 0, 4) \
    X(18, 128, 128, 64, 2, 2, 4, 3, 2, 2, 0, 4)  \
    X(19, 64, 64, 128, 1, 2, 5, -1, 4, 2, 0, 4)  \
    X(20, 32, 32, 128, 1, 1, 8, -1, 4, 2, 0, 2)  \
    X(21, 128, 128, 64, 1, 2, 4, -1, 2, 2, 0, 4) \
    X(22, 256, 256, 64, 4, 2, 2, 23, 1, 1, 4, 0, 12, 16) \
    X(23, 256, 128, 64, 2, 2, 3, -1, 4, 1, 0, 4, 0, 16) \
    X(24, 128, 128, 64, 1, 2, 4, -1, 2, 2, 0, 4, 0, 16) \
    X(25, 256, 192, 64, 4, 2, 2, 17, 1, 1, 4, 0, 10, 16)

#define FFN_NUM_VARIANTS 26

// (up variant, down variant) pairs compiled as a single-launch FFN (ffn_fused.hip); the two tiles
// of a pair have the same number of waves, and the up tile's rows are whole down tile rows.  The
// aligned mid-size, unaligned and DiT-size FFNs' Basic tile pairs (the unaligned one's up on
// variant 13, twelve-wave variant 18 having no eight-wave down to pair with).
#define FFN_FUSED_PAIRS(X) X(12, 21) X(13, 19) X(12, 17)


// launch roles of one variant
// (the split up roles: tiles split along K, FP32 partials, the activation applied by the last
// piece of each tile)
enum {
    FFN_ROLE_UP_ERF = 0,
    FFN_ROLE_UP_RATIONAL = 1,
    FFN_ROLE_DOWN_BASIC = 2,
    FFN_ROLE_DOWN_STREAMK = 3,
    FFN_ROLE_UP_SPLIT_ERF = 4,
    FFN_ROLE_UP_SPLIT_RATIONAL = 5,
    FFN_ROLE_UP_SILU = 6,
    FFN_ROLE_UP_SWIGLU = 7,       // tiles with wave tiles of whole 64-column block pairs only
    FFN_ROLE_UP_SPLIT_SILU = 8
};
