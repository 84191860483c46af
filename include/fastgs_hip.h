/*
 * fastgs_hip.h -- C ABI of libfastgs_hip.so, the MI355X (gfx950) FastGS
 * rasterizer.  Plain C: POD parameter/IO structs of raw device pointers,
 * element counts, and a hipStream_t passed as void*.  No torch types.
 *
 * Ownership: the caller allocates every output and workspace buffer (sizes
 * from the *_workspace_bytes queries); the library never allocates, frees or
 * retains device memory and never synchronises the stream.  The one exception
 * is fgs_inclusive_scan_u32_noalloc, whose state is a static device array of
 * the library (512.25 KiB per device).  Every output
 * element the reference zero-fills is written by the library on the stream
 * (kernels, never host memsets and never hipMemsetAsync).
 *
 * Alignment: arrays of rows of 2 floats ([N,2]) must be 8-byte aligned and
 * rows of 4 floats ([N,4]) 16-byte aligned, as hipMalloc returns them; the
 * kernels read and write such rows as one vector.
 *
 * Errors: every entry point returns FGS_OK (0) or a negative code; the
 * message of the last failure on the calling thread is fgs_last_error().
 *
 * Each entry point names the reference interface it replaces
 * (a1091150/fastgs_core, file:line).
 */
#ifndef FASTGS_HIP_H
#define FASTGS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FGS_OK 0
#define FGS_ERR_INVALID_ARGUMENT -1
#define FGS_ERR_LAUNCH -2
#define FGS_ERR_UNSUPPORTED -3

/* Thread-local message of the last error ("" if none). */
const char* fgs_last_error(void);

/* ABI version of this header (bumped on any struct/signature change or
 * addition). */
int32_t fgs_abi_version(void);

/* Launch events (measurement; no reference counterpart).  Asks the library
 * to record the caller's events `start` and `stop` (hipEvent_t, as void*) on
 * the launch stream directly before and after every launch of one kernel,
 * so that the kernel's own duration can be read with hipEventElapsedTime,
 * without the small kernels an entry point launches around it.  `kernel`
 * names the main kernel of one stage: "preprocess_fwd", "rasterize_fwd",
 * "rasterize_bwd", "preprocess_bwd", "loss_fwd" or "loss_bwd" (the SSIM map
 * kernels of fgs_l1_ssim_fwd / fgs_l1_ssim_bwd), or "preprocess_colour" (the
 * kernel of fgs_preprocess_colour_fwd; "preprocess_fwd" also names the kernel
 * of fgs_preprocess_geometry_fwd).  Both events NULL clears the
 * entry; one of them NULL, or an unknown name, is FGS_ERR_INVALID_ARGUMENT.
 * A process-wide setting read at each launch; the events must stay valid
 * until it is cleared. */
int32_t fgs_set_launch_events(const char* kernel, void* start, void* stop);

/* ------------------------------------------------------------------------ */
/* Preprocess.                                                               */
/* Replaces PreprocessParams/PreprocessKernelParams                          */
/* (fastgs_preprocess.h:13-55, fastgs_preprocess.cpp:21-38).                  */
/* ------------------------------------------------------------------------ */
typedef struct {
  int32_t P;                  /* number of Gaussians */
  int32_t degree;             /* SH degree (0..3; >3 treated as 3) */
  int32_t max_sh_coeffs;      /* sh.shape[1]: rest coefficients per Gaussian */
  int32_t image_width;
  int32_t image_height;
  int32_t grid_x;             /* ceil(W/16), at most 65535 */
  int32_t grid_y;             /* ceil(H/16), at most 65535 */
  int32_t use_cov3d_precomp;  /* geometry path: 1 = cov3d_precomp, 0 = scales+rotations */
  int32_t use_colors_precomp; /* colour path: 1 = colors_precomp, 0 = dc+sh */
  float scale_modifier;
  float mult;
  float tan_fovx;
  float tan_fovy;
} fgs_preprocess_params;

typedef struct {
  /* inputs (device, float32, contiguous); unused paths may be NULL */
  const float* means3d;        /* [P,3] */
  const float* dc;             /* [P,3]            (SH path) */
  const float* sh;             /* [P,max_sh,3]     (SH path) */
  const float* colors_precomp; /* [P,3]            (precomp colour path) */
  const float* opacities;      /* [P] */
  const float* scales;         /* [P,3] */
  const float* rotations;      /* [P,4] (r,x,y,z) */
  const float* cov3d_precomp;  /* [P,6] */
  const float* viewmatrix;     /* [16] column-major */
  const float* projmatrix;     /* [16] column-major */
  const float* campos;         /* [3] */
  const float* viewspace_in;   /* [P,4] */
  /* outputs (every element written) */
  int32_t* radii;              /* [P] */
  float* xys;                  /* [P,2] */
  float* depths;               /* [P] */
  float* cov3d;                /* [P,6] */
  float* rgb;                  /* [P,3] */
  float* conic_opacity;        /* [P,4] */
  uint32_t* tiles_touched;     /* [P] */
  uint8_t* clamped;            /* [P,3] bool */
  float* viewspace_out;        /* [P,4] */
  /* Optional (NULL: not written) super-tile records for fgs_binning_sorted,
   * no reference counterpart.  Super-tiles are 8x8 tiles, numbered row-major
   * on a grid ceil(grid_x/8) wide.  Record i is st_rec[4i..4i+3] =
   * (word, 0, lo, hi), in one of four forms:
   *  - word = x0 | y0 << 12 | 1u << 29 (compact): the Gaussian's tile
   *    rectangle has at most 8x8 tiles from tile (x0, y0), x0, y0 < 4096;
   *    lo | hi << 32 is its 8x8 board, bit (y - y0) * 8 + (x - x0) for tile
   *    (x, y); st_masks[4i..] not written;
   *  - word = bx | by << 12 | 1u << 31: the rectangle lies in the 2x2
   *    super-tiles from (bx, by), the super-tile of its corner;
   *    st_masks[4i + k] = its tiles in super-tile (bx + (k & 1), by + (k >> 1)),
   *    bit (y mod 8) * 8 + (x mod 8);
   *  - word = 1u << 30 (other rectangles, grids of at most 256 super-tiles):
   *    bit s of the 256-bit st_masks[4i..4i+3] marks each super-tile s
   *    holding one of its tiles;
   *  - word = 0: no tile touched (or a wide Gaussian on a larger grid);
   *    st_masks[4i..] not written.
   * Both set or both NULL, 16-byte aligned. */
  uint32_t* st_rec;            /* [P,4] */
  uint64_t* st_masks;          /* [P,4] */
  /* Training-step fusion (no reference counterpart; optional, NULL = off):
   * the raw parameters, activated here as the training scripts do
   * (train_scanner_fixed.py:523-536): scale = exp(log_scale), rotation =
   * q / (|q| + 1e-8), opacity = sigmoid(logit), bit-identical to
   * fgs_activations_fwd.  Each one set replaces its activated input, which
   * may then be NULL. */
  const float* log_scales;     /* [P,3] */
  const float* raw_rotations;  /* [P,4] */
  const float* opacity_logits; /* [P] */
} fgs_preprocess_fwd_io;

/* Replaces FastGSPreprocess::eval_gpu (fastgs_preprocess.cpp:81-169) /
 * fastgs_preprocess_forward_kernel (fastgs_preprocess.metal:384-484). */
int32_t fgs_preprocess_fwd(const fgs_preprocess_params* p, const fgs_preprocess_fwd_io* io,
                           void* stream);

/* fgs_preprocess_fwd in two halves (the same arguments, the same results):
 * the geometry half writes every output except rgb and clamped; the colour
 * half, queued after it (it reads radii), writes rgb and clamped.  The colour
 * half may run on another stream, ordered after the geometry half by an
 * event, so that it overlaps the binning that follows on the first stream.
 * No reference counterpart (the split of fastgs_preprocess.metal:384-484). */
int32_t fgs_preprocess_geometry_fwd(const fgs_preprocess_params* p,
                                    const fgs_preprocess_fwd_io* io, void* stream);
int32_t fgs_preprocess_colour_fwd(const fgs_preprocess_params* p, const fgs_preprocess_fwd_io* io,
                                  void* stream);

typedef struct {
  /* primals */
  const float* means3d;
  const float* scales;
  const float* rotations;
  const float* viewmatrix;
  const float* projmatrix;
  const float* campos;
  const float* sh;
  const float* cov3d_precomp;
  /* forward outputs */
  const float* cov3d_fwd;      /* [P,6] */
  const int32_t* radii;        /* [P] */
  const uint8_t* clamped;      /* [P,3] */
  /* cotangents of the preprocess outputs (NULL = zero) */
  const float* dL_dxys;            /* [P,2] */
  const float* dL_drgb;            /* [P,3] */
  const float* dL_dconic_opacity;  /* [P,4] */
  const float* dL_dcov3d;          /* [P,6] */
  const float* dL_dviewspace_out;  /* [P,4] */
  /* gradients (every element written; rows with radii <= 0 are zero) */
  float* dL_dmeans3d;          /* [P,3] */
  float* dL_ddc;               /* [P,3] */
  float* dL_dsh;               /* [P,max_sh,3] */
  float* dL_dcolors_precomp;   /* [P,3] */
  float* dL_dopacities;        /* [P] */
  float* dL_dscales;           /* [P,3] */
  float* dL_drotations;        /* [P,4] */
  float* dL_dviewspace_in;     /* [P,4] */
  /* Training-step fusion (no reference counterpart; optional, NULL = off):
   * the gradients of the raw parameters of the training scripts'
   * activations scale = exp(log_scale), rotation = q / (|q| + 1e-8),
   * opacity = sigmoid(logit) (train_scanner_fixed.py:523-536), written in
   * place of dL_dscales / dL_drotations / dL_dopacities (which may then be
   * NULL), bit-identical to fgs_activations_bwd applied to them.  quats_raw
   * are the raw quaternions q, act_opacities the sigmoid outputs; the scales
   * are `scales`.  dL_dlog_scales and dL_dquats need the scale / rotation
   * path (use_cov3d_precomp = 0).  With log_scales set the scales are
   * computed from it (scales may be NULL), with quats_raw set and rotations
   * NULL the rotations from quats_raw, and with opacity_logits set and
   * act_opacities NULL the opacities from the logits, as fgs_preprocess_fwd
   * does. */
  const float* quats_raw;      /* [P,4] */
  const float* act_opacities;  /* [P] */
  float* dL_dlog_scales;       /* [P,3] */
  float* dL_dquats;            /* [P,4] */
  float* dL_dlogits;           /* [P] */
  const float* log_scales;     /* [P,3] */
  const float* opacity_logits; /* [P] */
  /* Floats from one Gaussian's dL_dxys pair to the next (no reference
   * counterpart; 0 = 2, a [P,2] array).  4 reads the first two components of
   * a [P,4] array: the rasterize backward's dL_dviewspace, whose first two
   * components are dL_dmeans2d, so a caller that chains the two backwards
   * needs no copy.  At least 2 when not 0. */
  int64_t dL_dxys_stride;
} fgs_preprocess_bwd_io;

/* Replaces FastGSPreprocess::vjp -> FastGSPreprocessBackward::eval_gpu
 * (fastgs_preprocess.cpp:191-206, fastgs_preprocess_backward.cpp:89-185) /
 * fastgs_preprocess_backward_kernel (fastgs_preprocess_backward.metal:60-430). */
int32_t fgs_preprocess_bwd(const fgs_preprocess_params* p, const fgs_preprocess_bwd_io* io,
                           void* stream);

/* ------------------------------------------------------------------------ */
/* Scan / binning / sort / tile ranges.                                      */
/*                                                                            */
/* Bounded waits.  The scans and radix-sort passes are one-pass: each        */
/* 4096-element chunk waits for its predecessors' published sums (chunks are */
/* numbered in start order, so every wait ends).  Each wait is bounded as a  */
/* backstop; one that gives up uses a partial sum, which keeps every write   */
/* in bounds but makes the results invalid, and reports it in a wait-status  */
/* word: bit 0 a scan chunk, bit 1 a radix-pass look-back.  The entry points */
/* below take that word as `wait_status` (device, optional: NULL keeps it    */
/* inside the workspace); the call writes it (0 when every wait completed)   */
/* on the stream, and the caller reads it back with the results.             */
/* ------------------------------------------------------------------------ */

/* Polls of one bounded wait before it gives up (default 2^24); returns the
 * previous value.  A process-wide setting read when a call is issued.  0 makes
 * every wait give up at once without polling: every chunk after the first
 * reports it, so a test can drive the error path deterministically while
 * every kernel still runs to its end.  No reference counterpart. */
uint32_t fgs_set_wait_spin_limit(uint32_t limit);

/* Workspace for fgs_inclusive_scan_u32 over n elements. */
size_t fgs_scan_workspace_bytes(int64_t n);

/* out[i] = sum(in[0..i]) mod 2^32.  Replaces mx::cumsum(..., inclusive)
 * (binding.cpp:153,211).  in and out may alias.  wait_status: see above. */
int32_t fgs_inclusive_scan_u32(const uint32_t* in, uint32_t* out, int64_t n, void* workspace,
                               uint32_t* wait_status, void* stream);

/* fgs_inclusive_scan_u32 without a workspace: the scan's state lives in a
 * device array of the library (512.25 KiB per device, held until the process
 * ends), so the call allocates nothing and takes no workspace.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  n <= 2^28 (FGS_ERR_INVALID_ARGUMENT above).  Every call on a
 * device shares that device's array: calls that overlap on one device (other
 * streams, other threads) race and must be ordered by the caller. */
int32_t fgs_inclusive_scan_u32_noalloc(const uint32_t* in, uint32_t* out, int64_t n,
                                       uint32_t* wait_status, void* stream);

/* Gaussian-order duplication: for each Gaussian with tiles_touched > 0, the
 * keys (tile_id << 32 | float_bits(depth)) and values (index) of its touched
 * tiles at [point_offsets[i-1], ...).  keys/values are fully written (zero
 * where nothing is emitted).  Replaces FastGSBinning::eval_gpu
 * (fastgs_binning.cpp:59-106) / fastgs_duplicate_with_keys_kernel
 * (fastgs_binning.metal:182-213). */
int32_t fgs_duplicate_with_keys(int32_t P, const float* xys, const float* depths,
                                const uint32_t* point_offsets, const float* conic_opacity,
                                const uint32_t* tiles_touched, float mult, int32_t grid_x,
                                int32_t grid_y, int64_t num_rendered, uint64_t* keys_unsorted,
                                uint32_t* values_unsorted, void* stream);

/* Workspace for fgs_sort_pairs_u64 over n pairs. */
size_t fgs_sort_workspace_bytes(int64_t n);

/* Stable ascending LSD radix sort of (key, value) pairs on key bits
 * [begin_bit, end_bit).  Output in keys_out/values_out.  Replaces
 * mx::argsort + 2x mx::take (binding.cpp:195-197); ties keep input order.
 * values_in NULL: the values are the input positions.  wait_status: see
 * above. */
int32_t fgs_sort_pairs_u64(const uint64_t* keys_in, const uint32_t* values_in, uint64_t* keys_out,
                           uint32_t* values_out, int64_t n, int32_t begin_bit, int32_t end_bit,
                           void* workspace, uint32_t* wait_status, void* stream);

/* ranges[T][2] and bucket_count[T] from (sorted) 64-bit keys with the exact
 * semantics of fastgs_identify_tile_ranges_kernel and
 * fastgs_per_tile_bucket_count_kernel (fastgs_tile_prep.metal:10-53); keys
 * with tile 0xFFFFFFFF or tile >= T are ignored.  Replaces
 * FastGSTilePrep::eval_gpu (fastgs_tile_prep.cpp:48-99). */
int32_t fgs_tile_ranges(const uint64_t* keys, int64_t num_rendered, int32_t num_tiles,
                        uint32_t* ranges, uint32_t* bucket_count, void* stream);

/* Fused binning of the rasterize_gaussians path (binding.cpp:175-212):
 * duplicate -> stable sort on (tile, depth) -> tile ranges -> bucket counts
 * -> bucket offsets.  Produces exactly the arrays of the reference path. */
typedef struct {
  int32_t P;
  int32_t grid_x;
  int32_t grid_y;
  int64_t num_rendered; /* K = point_offsets[P-1] */
  float mult;
  /* inputs */
  const float* xys;
  const float* depths;
  const float* conic_opacity;
  const uint32_t* tiles_touched;
  /* outputs */
  uint64_t* point_list_keys;  /* [K] sorted */
  uint32_t* point_list;       /* [K] sorted */
  uint32_t* ranges;           /* [T,2] */
  uint32_t* bucket_count;     /* [T] */
  uint32_t* bucket_offsets;   /* [T] inclusive */
  void* workspace;            /* fgs_binning_workspace_bytes(P, K, T) */
  /* NULL (the Gaussians are sorted by depth here), or the depth workspace of
   * an fgs_depth_order call on the same P, depths and tiles_touched that is
   * ordered before this call (same stream, or an event). */
  const void* depth_order;
  /* NULL, or the super-tile records fgs_preprocess_fwd wrote for these
   * Gaussians (same grid): Gaussians with a record skip their tile walks. */
  const uint32_t* st_rec;
  const uint64_t* st_masks;
  /* NULL, or a device word the call writes with the wait status (see above)
   * of its own waits and of the depth order it consumes (depth_order, or the
   * one it runs itself), after them in stream order. */
  uint32_t* wait_status;
  /* NULL, or host memory the device can write (pinned) for one 64-bit word
   * (no reference counterpart: the read of B at binding.cpp:209-212 without
   * a copy).  When num_tiles > 0 the call's bucket scan writes
   * (wait status << 32) | B there, B = bucket_offsets[T-1], as one store at
   * system scope, once both are known (before the call's last kernel).  The
   * caller sets the word to a value whose low half is 0xFFFFFFFF first and
   * reads it once it has changed. */
  uint64_t* host_result;
} fgs_binning_io;

size_t fgs_binning_workspace_bytes(int32_t P, int64_t num_rendered, int32_t num_tiles);
int32_t fgs_binning_sorted(const fgs_binning_io* io, void* stream);

/* The first stage of fgs_binning_sorted on its own: the visible Gaussians
 * (tiles_touched > 0) ordered by depth bits (stable).  The order buffer holds
 * them in its first nvis entries, followed by 0xFFFFFFFF sentinels up to P
 * (the culled Gaussians are dropped, so it is not a permutation of [0, P));
 * the count nvis stays in depth_workspace for fgs_binning_sorted.  It needs
 * only P, so a caller can enqueue it before the blocking read of
 * K = point_offsets[P-1] (binding.cpp:25-31,153-154) and the GPU sorts while
 * the host waits; the result is passed as fgs_binning_io.depth_order.  No
 * reference counterpart of its own: it is the depth half of the argsort at
 * binding.cpp:195-197.  depth_workspace: fgs_depth_order_workspace_bytes(P),
 * 256-byte aligned, no initial contents required.  The sort's wait status
 * stays in the workspace and is reported by the fgs_binning_sorted call that
 * consumes it. */
size_t fgs_depth_order_workspace_bytes(int32_t P);
int32_t fgs_depth_order(int32_t P, const float* depths, const uint32_t* tiles_touched,
                        void* depth_workspace, void* stream);

/* ------------------------------------------------------------------------ */
/* Rasterize.                                                                */
/* Replaces RasterizeParams/RasterizeKernelParams (fastgs_rasterize.h:14-51, */
/* fastgs_rasterize.cpp:20-29).                                              */
/* ------------------------------------------------------------------------ */
typedef struct {
  int32_t image_width;
  int32_t image_height;
  int32_t num_channels;   /* colour row stride; min(num_channels,3) blended */
  int32_t num_tiles;
  int64_t bucket_sum;     /* B */
  int32_t get_flag;
  int32_t write_sampled;  /* 1: also write sampled_t / sampled_ar */
  int32_t num_points;     /* P: Gaussians; list entries >= P are treated as empty */
  int64_t list_len;       /* K: length of point_list; ranges are clamped to it */
} fgs_raster_params;

typedef struct {
  const uint32_t* ranges;          /* [T,2] */
  const uint32_t* point_list;      /* [K] */
  const uint32_t* bucket_offsets;  /* [T] inclusive */
  const float* means2d;            /* [P,2] */
  const float* colors;             /* [P,num_channels] */
  const float* conic_opacity;      /* [P,4] */
  const float* background;         /* [num_channels] */
  const int32_t* metric_map;       /* [H*W] (read when get_flag) */
  uint32_t* bucket_to_tile;        /* [B] */
  float* sampled_t;                /* [B*256]      (when write_sampled) */
  float* sampled_ar;               /* [B][C][256]  (when write_sampled) */
  float* final_t;                  /* [H*W] */
  uint32_t* n_contrib;             /* [H*W] */
  uint32_t* max_contrib;           /* [T] */
  float* pixel_colors;             /* [C,H*W] */
  float* out_color;                /* [C,H*W] */
  int32_t* metric_count;           /* [P] (zeroed and accumulated when get_flag) */
  /* NULL, or [H*W]: each pixel's loop iterations under the reference loop
   * (fastgs_rasterize.metal:100-131: the splats it visits, the one it stops
   * at included), a measurement output with no reference counterpart. */
  uint32_t* n_iter;
} fgs_raster_fwd_io;

/* Replaces FastGSRasterize::eval_gpu (fastgs_rasterize.cpp:91-169) /
 * fastgs_render_forward_kernel (fastgs_rasterize.metal:25-159). */
int32_t fgs_rasterize_fwd(const fgs_raster_params* p, const fgs_raster_fwd_io* io, void* stream);

typedef struct {
  const uint32_t* ranges;
  const uint32_t* point_list;
  const float* means2d;
  const float* colors;
  const float* conic_opacity;
  const float* background;
  const float* final_t;         /* [H*W] from the forward */
  const uint32_t* n_contrib;    /* [H*W] from the forward */
  const uint32_t* max_contrib;  /* [T] from the forward */
  const float* dL_dout_color;   /* [C,H*W] */
  float* dL_dmeans2d;           /* [P,2], or NULL: not written (it equals the first two
                                   components of dL_dviewspace, which a caller may read in
                                   place; fgs_preprocess_bwd_io.dL_dxys_stride = 4) */
  float* dL_dcolors;            /* [P,num_channels] */
  float* dL_dconic_opacity;     /* [P,4] */
  float* dL_dviewspace;         /* [P,4] */
  uint32_t* tile_order;         /* [T] scratch, or NULL.  When set (and T <= 65536) the tiles
                                   are walked heaviest first by max_contrib, which shortens the
                                   launch's tail; NULL walks them in index order.  The result is
                                   the same either way, up to the order of float atomic adds. */
} fgs_raster_bwd_io;

/* Gradients of the blend w.r.t. means2d (scaled by (W/2,H/2)), colours,
 * conic/opacity and the viewspace dummy (x, y, |x|, |y|).  Every output
 * element is written.  Replaces FastGSRasterize::vjp ->
 * FastGSRasterizeBackward::eval_gpu (fastgs_rasterize.cpp:191-206,
 * fastgs_rasterize_backward.cpp:85-168) / fastgs_render_backward_kernel
 * (fastgs_rasterize_backward.metal:24-278). */
int32_t fgs_rasterize_bwd(const fgs_raster_params* p, const fgs_raster_bwd_io* io, void* stream);

/* ------------------------------------------------------------------------ */
/* Training-step loss (the caller side of the path, reference               */
/* scripts/train_scanner_fastgs.py:911-966): L = w_l1 mean|x-y| +             */
/* w_ssim (1 - mean SSIM(x,y)), 11x11 Gaussian window (sigma 1.5), zero       */
/* padding, per channel; x, y are [C,H,W] float32.                            */
/* ------------------------------------------------------------------------ */
size_t fgs_l1_ssim_workspace_bytes(int32_t C, int32_t H, int32_t W);

/* Writes the loss scalar to *loss (device).  When dmaps != NULL ([3,C,H,W])
 * also writes the per-pixel partial derivatives the backward needs. */
int32_t fgs_l1_ssim_fwd(const float* img, const float* tgt, int32_t C, int32_t H, int32_t W,
                        float w_l1, float w_ssim, float* loss, float* dmaps, void* workspace,
                        void* stream);

/* dimg = grad_out[0] * dL/dimg (grad_out: device scalar, NULL = 1). */
int32_t fgs_l1_ssim_bwd(const float* img, const float* tgt, const float* dmaps,
                        const float* grad_out, int32_t C, int32_t H, int32_t W, float w_l1,
                        float w_ssim, float* dimg, void* stream);

/* The pointwise losses of the FastGS training script's loss_fn
 * (scripts/train_scanner_fastgs.py:911-966): *loss = mean |x - y| (mode 0)
 * or mean (x - y)^2 (mode 1) over n floats, terms summed in double in a fixed
 * order; the backward writes dx = g * sign(x - y) / n or g * 2 (x - y) / n
 * (g = *grad_out, 1 when NULL).  No counterpart in the reference library (its
 * script computes them with MLX). */
size_t fgs_pointwise_loss_workspace_bytes(int64_t n);
int32_t fgs_pointwise_loss_fwd(const float* x, const float* y, int64_t n, int32_t mode,
                               void* workspace, float* loss, void* stream);
int32_t fgs_pointwise_loss_bwd(const float* x, const float* y, int64_t n, int32_t mode,
                               const float* grad_out, float* dx, void* stream);

/* ------------------------------------------------------------------------ */
/* Training-step glue.  No counterpart in the reference library: the         */
/* reference's training scripts do these in MLX (activations                 */
/* scripts/train_scanner_fixed.py:523-536; optimizer                          */
/* scripts/train_scanner_fastgs.py:77-182).                                   */
/* ------------------------------------------------------------------------ */

/* scales = exp(log_scales) [P,3], rotations = q / (|q| + 1e-8) [P,4],
 * opacities = sigmoid(opacity_logits) [P].  Each input may be NULL (its output
 * is then not written). */
int32_t fgs_activations_fwd(int32_t P, const float* log_scales, const float* quats,
                            const float* opacity_logits, float* scales, float* rotations,
                            float* opacities, void* stream);

/* Backward of fgs_activations_fwd from the gradients of the activated
 * tensors (NULL = zero): d_log_scales needs scales, d_quats needs quats,
 * d_logits needs opacities (the forward's outputs / inputs).  A NULL output
 * is not written. */
int32_t fgs_activations_bwd(int32_t P, const float* quats, const float* scales,
                            const float* opacities, const float* d_scales,
                            const float* d_rotations, const float* d_opacities,
                            float* d_log_scales, float* d_quats, float* d_logits, void* stream);

/* One in-place Adam step over n floats (step >= 1 counts this update):
 * m = b1 m + (1-b1) g; v = b2 v + (1-b2) g^2;
 * bias_correction == 0 (MLX's Adam default): p -= lr m / (sqrt(v) + eps);
 * bias_correction != 0: p -= lr/(1-b1^step) m / (sqrt(v)/sqrt(1-b2^step) + eps). */
int32_t fgs_adam_step(float* param, const float* grad, float* exp_avg, float* exp_avg_sq,
                      int64_t n, float lr, float beta1, float beta2, float eps, int32_t step,
                      int32_t bias_correction, void* stream);

/* Up to 8 tensors in one launch, each with its own learning rate and step
 * count, the update of fgs_adam_step.  No counterpart in the reference: its
 * MLX optimizer steps each array on its own (train_scanner_fastgs.py:77-182);
 * one launch for the six Gaussian parameter tensors saves five. */
typedef struct {
  float* param;
  const float* grad;
  float* exp_avg;
  float* exp_avg_sq;
  int64_t n;
  float lr;
  int32_t step;
} fgs_adam_group;
int32_t fgs_adam_step_multi(const fgs_adam_group* groups, int32_t count, float beta1, float beta2,
                            float eps, int32_t bias_correction, void* stream);

/* Fill a u32 buffer with a value on the stream (a kernel, graph-safe). */
int32_t fgs_fill_u32(uint32_t* dst, uint32_t value, int64_t n, void* stream);

/* ------------------------------------------------------------------------ */
/* Densification and pruning.  No counterpart in the reference library: the  */
/* reference's FastGS training script does these on the host with numpy      */
/* (scripts/train_scanner_fastgs.py: scores :279-340, statistics :391-405,    */
/* clone/split/prune :470-616 and :661-742, final prune :745-793, opacity     */
/* cap/reset :619-658).  Rows are the reference's parameter rows; exp/log are */
/* the library's deterministic ones.  Random numbers are inputs.              */
/* ------------------------------------------------------------------------ */

/* Gradient statistics of one step (:391-405): for rows with radii > 0,
 * max_radii2d = max(max_radii2d, radii), grad_accum += |d_viewspace[:2]|,
 * grad_accum_abs += |d_viewspace[2:]|, denom += 1; tmp_radii = radii on
 * every row.  d_viewspace: the [P,4] viewspace gradient. */
int32_t fgs_densify_stats(int32_t P, const int32_t* radii, const float* d_viewspace,
                          float* max_radii2d, float* grad_accum, float* grad_accum_abs,
                          float* denom, int32_t* tmp_radii, void* stream);

/* Thresholds of densify_and_prune_fastgs (:661-742), as float32. */
typedef struct {
  float grad_thresh;          /* args.grad_thresh */
  float grad_abs_thresh;      /* args.grad_abs_thresh */
  float clone_max_scale;      /* args.dense * scene_extent */
  float importance_threshold; /* args.importance_score_threshold */
  float min_opacity;          /* args.min_opacity */
  float max_screen_size;      /* args.max_screen_size (<= 0: off) */
  float world_max_scale;      /* args.max_world_scale_factor * scene_extent (<= 0: off) */
  int32_t split_factor;       /* args.split_factor */
} fgs_densify_params;

/* Clone and split flags (u32 0/1) of the P current rows: clone = importance >
 * threshold && max scale <= clone_max_scale && |grad_accum/max(denom,1)| >=
 * grad_thresh; split = importance > threshold && max scale > clone_max_scale
 * && |grad_accum_abs/max(denom,1)| >= grad_abs_thresh. */
int32_t fgs_densify_classify(int32_t P, const fgs_densify_params* prm, const float* grad_accum,
                             const float* grad_accum_abs, const float* denom,
                             const float* log_scales, const float* importance,
                             uint32_t* clone_flag, uint32_t* split_flag, void* stream);

/* The P2 = P - ns + nc + ns * split_factor pre-prune rows, from the
 * inclusive scans of the flags (nc, ns: their totals): the rows that are not
 * split sources in order, then the clones, then split_factor children per
 * source, consecutive.  l2_src: source row; l2_kind: 0 kept, 1 clone, 2 split
 * child; l2_child: the child's row in the normals array, else -1. */
int32_t fgs_densify_layout(int32_t P, int32_t split_factor, const uint32_t* clone_incl,
                           const uint32_t* split_incl, int32_t* l2_src, int32_t* l2_kind,
                           int32_t* l2_child, void* stream);

/* Prune candidates of the P2 pre-prune rows (opacity < min_opacity, screen
 * size when nothing was appended, world scale) and their removal keys: for a
 * candidate, the float bits of (-log(1 - u)) * (1e-6 + (1 - pruning_score))
 * (u: uniforms[r] in [0,1)), whose k smallest are a weighted sample without
 * replacement with weights 1 / (1e-6 + (1 - score)); otherwise 0xFFFFFFFF.
 * pruning_score NULL: all keys 0xFFFFFFFF.  l2_src / l2_kind NULL: identity.
 * Appended rows take their source's score. */
int32_t fgs_densify_prune_keys(int32_t P2, const fgs_densify_params* prm, int32_t any_appended,
                               const int32_t* l2_src, const int32_t* l2_kind,
                               const float* opacity_logits, const float* log_scales,
                               const float* max_radii2d, const float* pruning_score,
                               const float* uniforms, uint64_t* keys, uint32_t* candidate,
                               void* stream);

/* keep[sorted_rows[j]] = (j >= k): the first k rows of a sorted order are
 * removed. */
int32_t fgs_densify_select(int32_t P2, int64_t k, const uint32_t* sorted_rows, uint32_t* keep,
                           void* stream);

/* keep[sorted_rows[j]] = (j < k): the first k rows of a sorted order kept. */
int32_t fgs_densify_keep_first(int32_t P, int64_t k, const uint32_t* sorted_rows, uint32_t* keep,
                               void* stream);

/* out[i] = !in[i] (u32 flags). */
int32_t fgs_invert_flags(int32_t n, const uint32_t* in, uint32_t* out, void* stream);

/* rows[keep_incl[r] - 1] = r for the kept rows (keep_incl: inclusive scan of
 * keep). */
int32_t fgs_densify_compact(int32_t P2, const uint32_t* keep, const uint32_t* keep_incl,
                            int32_t* rows, void* stream);

/* The new row set: new row f comes from pre-prune row rows[f] (NULL:
 * identity), which comes from source row l2_src (NULL with l2_kind: identity,
 * all kept).  Parameters and their Adam moments (exp_avg / exp_avg_sq in the
 * order means3d, features_dc, features_rest, opacity_logits, log_scales,
 * rotations; NULL entries skipped) are copied from the source, moments of
 * appended rows are zero; statistics are copied, or zero when reset_stats.
 * Split children: mean + R(q)(exp(log_scale) * z) with z = normals[l2_child]
 * and log scales log(exp(ls) / (0.8 split_factor)) (:560-583).  opacity_cap
 * > 0: every opacity logit becomes logit(min(sigmoid(x), cap)) and the
 * opacity moments restart at zero (:619-637).  Sources and destinations must
 * not overlap. */
typedef struct {
  int32_t P_new;
  int32_t sh_row;        /* floats per features_rest row */
  int32_t split_factor;
  int32_t reset_stats;
  float opacity_cap;
  const int32_t* rows;
  const int32_t* l2_src;
  const int32_t* l2_kind;
  const int32_t* l2_child;
  const float* normals;  /* [children, 3] */
  const float* means3d;
  const float* features_dc;
  const float* features_rest;
  const float* opacity_logits;
  const float* log_scales;
  const float* rotations;
  const float* exp_avg[6];
  const float* exp_avg_sq[6];
  const float* max_radii2d;
  const float* grad_accum;
  const float* grad_accum_abs;
  const float* denom;
  const int32_t* tmp_radii;
  float* d_means3d;
  float* d_features_dc;
  float* d_features_rest;
  float* d_opacity_logits;
  float* d_log_scales;
  float* d_rotations;
  float* d_exp_avg[6];
  float* d_exp_avg_sq[6];
  float* d_max_radii2d;
  float* d_grad_accum;
  float* d_grad_accum_abs;
  float* d_denom;
  int32_t* d_tmp_radii;
} fgs_densify_build_io;
int32_t fgs_densify_build(const fgs_densify_build_io* io, void* stream);

/* logit(min(sigmoid(x), cap)) on every opacity logit, and the opacity Adam
 * moments (NULL: skipped) set to zero (cap_opacity_logits /
 * reset_opacity_logits, :619-658). */
int32_t fgs_opacity_cap(int32_t P, float cap, float* opacity_logits, float* exp_avg,
                        float* exp_avg_sq, void* stream);

/* The scoring render's metric map (:300-304): l = mean over channels of
 * |pred - target| per pixel ([C, HW] arrays), metric_map = (l - min) /
 * max(max - min, 1e-6) > loss_thresh; photometric_loss (device float) = mean
 * |pred - target|, summed in double. */
size_t fgs_metric_map_workspace_bytes(int64_t HW);
int32_t fgs_metric_map(int32_t C, int64_t HW, const float* pred, const float* target,
                       float loss_thresh, void* workspace, int32_t* metric_map,
                       float* photometric_loss, void* stream);

/* counts += metric_count; score += photometric_loss * metric_count
 * (:306-320). */
int32_t fgs_score_accumulate(int32_t P, const int32_t* metric_count,
                             const float* photometric_loss, float* counts, float* score,
                             void* stream);

/* pruning = (score - min) / max(max - min, 1e-6); importance (NULL: not
 * written) = floor(counts / max(n_cams, 1)) (:334-339).  minmax_ws: 2
 * words. */
int32_t fgs_score_finalize(int32_t P, int32_t n_cams, const float* counts, const float* score,
                           float* importance, float* pruning, uint32_t* minmax_ws, void* stream);

/* Final prune mask (:754-757): opacity < min_opacity || score > score_thresh,
 * and keys that sort ascending in order of descending opacity - score (the
 * keep priority of :771-776; ties keep row order). */
int32_t fgs_final_prune_mask(int32_t P, float min_opacity, float score_thresh,
                             const float* opacity_logits, const float* pruning_score,
                             uint32_t* prune, uint64_t* priority_keys, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTGS_HIP_H */
