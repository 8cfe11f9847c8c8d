#pragma once

/*
 * C-ABI of libkvpersist.so, upstream motion producer: dense Farneback optical
 * flow between consecutive gray frames and the per-tile change rates the
 * gating policies rank (reference: traces/gen_motion_from_video.py:61-67,
 * 104-126), gfx950 native.
 *
 * The reference calls OpenCV from Python:
 *   flow = cv2.calcOpticalFlowFarneback(prev, next, None, pyr_scale=0.5,
 *            levels=3, winsize=15, iterations=3, poly_n=5, poly_sigma=1.2,
 *            flags=0)                      (gen_motion_from_video.py:108-111)
 * then the magnitude, its mean over latent-grid cells and over row-major
 * tiles of cells (:112-121). The entry points below replace those calls with
 * the same argument meaning; the flow follows OpenCV 4.x's published
 * Farneback algorithm (modules/video/src/optflowgf.cpp).
 *
 * Conventions are those of kvp_c_api.h: device pointers owned by the caller
 * (16-byte aligned), int returns 0 = success with the text in
 * kvp_last_error(), `stream` is a hipStream_t (NULL = null stream).
 * Frames are uint8 gray [height, width] row-major; flow is fp32
 * [height, width, 2] holding (dx, dy) per pixel, as cv2 returns it.
 */

#include "kvp_c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Device workspace kvp_farneback_flows needs for num_frames frames
 * (kvp_farneback_flow: num_frames = 2). -1 on bad arguments. */
long kvp_farneback_workspace_bytes(int num_frames, int width, int height,
                                   double pyr_scale, int levels);

/* cv2.calcOpticalFlowFarneback(frames[p], frames[p + 1], None, pyr_scale,
 * levels, winsize, iterations, poly_n, poly_sigma, flags) for every pair
 * p = 0 .. num_frames-2 of a clip (reference:
 * traces/gen_motion_from_video.py:107-115), in one pass: each frame's
 * pyramid and polynomial expansion are computed once and shared by its two
 * pairs. frames uint8 [num_frames, height, width]; flows fp32
 * [num_frames-1, height, width, 2].
 * Supported: flags 0 (zero initial flow, box window), 0 < pyr_scale < 1,
 * winsize 1..49, poly_n 1..8, sides 10..8192, 2..4096 frames. */
int kvp_farneback_flows(const unsigned char* frames, int num_frames, int width,
                        int height, double pyr_scale, int levels, int winsize,
                        int iterations, int poly_n, double poly_sigma,
                        int flags, void* workspace, long workspace_bytes,
                        float* flows, void* stream);

/* One pair: cv2.calcOpticalFlowFarneback(prev, next, None, ...) ->
 * flow fp32 [height, width, 2] (reference: gen_motion_from_video.py:110). */
int kvp_farneback_flow(const unsigned char* prev, const unsigned char* next,
                       float* flow, int width, int height, double pyr_scale,
                       int levels, int winsize, int iterations, int poly_n,
                       double poly_sigma, int flags, void* workspace,
                       long workspace_bytes, void* stream);

/* kvp_farneback_flows with an event after every kernel launch, for
 * measurement (no counterpart in the reference, whose flow is a cv2 call):
 * launch i took launch_ms[i] on `stream`; launch_kind[i] is 0 pre-blur rows,
 * 1 pre-blur columns + resize, 2 polynomial expansion, 3 first matrix update
 * of a level (initial flow), 4 box filter + flow solve, 5 matrix update;
 * launch_level[i] is the pyramid level (0 = full size). Synchronises the
 * stream. *count receives the number of launches (an error if > capacity). */
int kvp_farneback_profile(const unsigned char* frames, int num_frames,
                          int width, int height, double pyr_scale, int levels,
                          int winsize, int iterations, int poly_n,
                          double poly_sigma, int flags, void* workspace,
                          long workspace_bytes, float* flows, float* launch_ms,
                          int* launch_kind, int* launch_level, int capacity,
                          int* count, void* stream);

/* Per-pair change rates (reference: gen_motion_from_video.py:61-67,112-121):
 * mag = |flow|; cell_maps fp32 [pairs, grid_rows, grid_cols] = mean of mag
 * over (height/grid_rows) x (width/grid_cols) pixel cells; change fp64
 * [pairs, tiles] = mean of each run of tile_tokens cells in row-major order
 * (tiles = ceil(grid_rows*grid_cols / tile_tokens), the last run may be
 * shorter). The grid must divide the frame. */
int kvp_motion_change_rates(const float* flows, int pairs, int width,
                            int height, int grid_rows, int grid_cols,
                            int tile_tokens, float* cell_maps, double* change,
                            void* stream);

#ifdef __cplusplus
}
#endif
