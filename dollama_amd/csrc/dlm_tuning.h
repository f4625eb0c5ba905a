/*
 * dlm_tuning.h - tile-selection overrides of libdlm_hip.so's GEMM / conv
 * dispatch, for tile sweeps and the tile-coverage tests.  Internal: not part
 * of the product ABI in include/ and not a counterpart of any reference
 * interface; the default (automatic) selection needs none of them.  The
 * symbols are exported so tests and tuning scripts can bind them.
 */
#ifndef DLM_TUNING_H
#define DLM_TUNING_H

#ifdef __cplusplus
extern "C" {
#endif

/* Tuning aids: force the MFMA GEMM / conv tile configuration, and the
 * split-K factor, for every following launch made by the calling thread
 * (0 = automatic).  Tiles 1-7: the register-staged core (128x128, 128x64, 64x64,
 * 128x32, 256x128, 128x256, 256x256); 8-25: the LDS-DMA core
 * (BMxBN, wave tile, ring depth) = 8 128x128 64x64 2, 9 128x64 64x32 2,
 * 10 128x128 64x64 4, 11 128x64 64x32 4, 12 64x128 32x64 2,
 * 13 256x128 128x64 2, 14 128x128 64x32 4, 15 128x128 64x32 2,
 * 16 256x128 64x64 2, 17 128x128 32x64 4, 18 128x128 64x32 5,
 * 19 256x128 64x64 3, 20 128x64 64x32 6, 21 256x160 64x80 3,
 * 22 128x160 32x80 3, 23 128x160 64x80 2, 24 128x160 32x80 4,
 * 25 64x160 32x80 2, 26 128x80 16x80 5; 27-34 the same core with the next
 * slice's first fragments read during the current slice's last MFMAs:
 * 27 128x80 16x80 5, 28 256x160 64x80 3, 29 128x128 64x32 2,
 * 30 128x160 32x80 4, 31 128x160 32x80 3, 32 256x128 64x64 3,
 * 33 128x128 64x32 4, 34 128x64 64x32 2; 35-39 ring stages of two K
 * slices under one barrier (BMxBN, wave tile, stages): 35 128x80 16x80 3,
 * 36 128x80 16x80 2, 37 128x160 32x80 2, 38 128x128 64x32 2,
 * 39 128x64 64x32 3; 40 128x128 32x64 2 and 41 256x160 32x160 3 with the
 * next slice's first fragments read early; 42 128x16 16x16 3 and 43 64x16
 * 16x16 3 (outputs of at most 16 columns); 44 192x160 48x80 3 (at most 192
 * rows, e.g. the text tokens' K/V projection).  Splits apply to the LDS-DMA core
 * only. */
int dlm_gemm_force_tile(int tile_id);
/* Same override for GEMMs / convs of one shape (M, N = output columns,
 * K = reduction length); tile 0 and splits 0 remove it, M = N = K = 0 clears
 * every override.  Like every tuning aid here it is thread-local: it steers
 * only launches made by the calling thread. */
int dlm_gemm_override_shape(int M, int N, int K, int tile_id, int splits);
int dlm_gemm_force_split(int splits);
/* Tuning aid: select alternative tile heuristics (0 = default; bit 0 = no
 * 160-column / split-K rules; bit 1 = no fragment-prefetch forms, four
 * splits for 256x160 grids that fill the chip). */
int dlm_gemm_set_variant(int variant);

/* Counter calibration: `blocks` workgroups of 4 waves, each wave `iters`
 * rounds of eight v_mfma_f32_32x32x16_f16 on register operands (no memory
 * traffic in the loop): blocks * 4 * iters * 8 * 32768 FLOP per launch,
 * from which a profiler's MFMA counters can be read against a known rate.
 * out receives blocks * 256 floats. */
int dlm_mfma_probe(int blocks, int iters, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DLM_TUNING_H */
