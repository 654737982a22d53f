/*
 * wmma_calib.h -- calibration kernels (libwmma_calib.so), used by bench.py to measure what
 * the MI355X itself sustains: the matrix pipe's rate with no memory traffic, and a plain
 * streaming read.  They are measuring instruments, not part of the wmma_ops path, and have
 * no counterpart in the reference.  Return 0 on success, nonzero on a bad argument (1, 2)
 * or a launch error (5).  Asynchronous on `stream` (a hipStream_t as void*).
 */
#ifndef WMMA_CALIB_H
#define WMMA_CALIB_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* `workgroups` workgroups of 4 waves; every wave issues `iters` (even) x 8 independent
 * v_mfma_f32_32x32x16_f16 on register operands, each MFMA of a round on a different pair
 * of the lane's 8 A and 8 B fragments.  operands: device memory of workgroups * 256 * 16
 * 16-byte fragments (random data makes the operand bits switch as in a GEMM), or NULL for
 * constant operands.  sink: device float[workgroups] (never written in practice; it keeps
 * the work observable). */
int wmma_calib_mfma_ceiling(int workgroups, int iters, const void* operands, float* sink,
                            void* stream);
/* FLOPs one wmma_calib_mfma_ceiling launch performs (2 per multiply-add). */
double wmma_calib_mfma_ceiling_flops(int workgroups, int iters);

/* LDS read rate: `workgroups` workgroups of 8 waves, each wave reading 8 KB of a 64 KB LDS
 * buffer per iteration, `iters` iterations.  mode 0: ds_read_b128, 1 KB contiguous per
 * instruction; 1: ds_read_b64_tr_b16, 512 contiguous bytes per instruction; 2:
 * ds_read_b64_tr_b16 in the flash forward's V-fragment pattern (D = 128).  Other modes
 * return 2.  sink: device float[workgroups]. */
int wmma_calib_lds_read(int mode, int workgroups, int iters, float* sink, void* stream);
/* Bytes one wmma_calib_lds_read launch reads from LDS. */
double wmma_calib_lds_read_bytes(int workgroups, int iters);

/* Reads `bytes` (a multiple of 16; src 16-byte aligned) once: workgroups of 8 waves, each
 * wave `loads_per_wave` (2, 4 or 8) 1 KB nontemporal loads of one contiguous run.
 * sink: device float[bytes / (8 KB * loads_per_wave) + 1]. */
int wmma_calib_read_stream(const void* src, size_t bytes, int loads_per_wave, float* sink,
                           void* stream);

/* The same with the launch shape chosen: workgroups of `threads` threads, every lane
 * `loads_per_lane` 16-byte loads (one contiguous run of threads * loads_per_lane * 16 bytes
 * per workgroup).  Shapes (threads x loads): 64x16, 256x{2,4,8}, 512x{2,4,8}, 1024x{2,4};
 * others return 2.  sink: device float[bytes / (16 * threads * loads_per_lane) + 1]. */
int wmma_calib_read_stream_shape(const void* src, size_t bytes, int threads, int loads_per_lane,
                                 float* sink, void* stream);

/* The activation stage of the small-M LDS-DMA GEMMs, alone: `workgroups` workgroups of
 * `waves` (4 or 8) waves each copy `iters` 64-row x 128-byte blocks (rows `row_bytes`
 * apart; `strided` = 0: contiguous 8 KB blocks of the same buffer) from an L2-resident
 * buffer of `bytes` (>= 128 rows) into LDS by buffer_load ... lds, `depth` (1, 4 or 8) - 1
 * blocks in flight.  Bytes moved: wmma_calib_l2_stage_bytes. */
int wmma_calib_l2_stage(int waves, int depth, int strided, const void* src, size_t bytes,
                        size_t row_bytes, int workgroups, int iters, float* sink, void* stream);
double wmma_calib_l2_stage_bytes(int workgroups, int iters);

#ifdef __cplusplus
}
#endif

#endif /* WMMA_CALIB_H */
