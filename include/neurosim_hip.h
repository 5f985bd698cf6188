/*
 * neurosim_hip.h -- C ABI of the MI355X (gfx950) dendritic tick library.
 *
 * This library replaces the pybind11 module `neurosim_gpu_native` that the
 * reference JIT-builds from csrc/bindings.cpp + csrc/compartmental.cu.  Every
 * entry point takes plain device pointers, sizes and strides (no framework
 * types), validates its arguments on the host, returns NS_OK or an error code,
 * and never synchronises the host.  Kernels are enqueued on the caller's
 * stream (a hipStream_t passed as void*; NULL means the legacy default
 * stream).  Nothing here allocates device memory: outputs and workspaces are
 * owned by the caller.
 *
 * Dynamics implemented by the tick (one (neuron n, column b) pair):
 *   j      = sum_e W[n, col[e]] * s[b, col[e]]            (CSR row n)
 *   d'     = rho_d*d + (1-rho_d)*tanh(j + dendritic_drive)
 *   u      = (1-c)*j + c*d' - k*a
 *   s'     = clamp(alpha*s + (1-alpha)*(gain*tanh(u + drive)), 0, 1)
 *   a'     = rho_a*a + (1-rho_a)*s'
 * with the parameter order of the reference (native_compartmental.py:20-23):
 *   [alpha, gain, dendrite_decay (rho_d), adaptation_decay (rho_a),
 *    coupling (c), adaptation_strength (k)].
 */
#ifndef NEUROSIM_HIP_H
#define NEUROSIM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NS_ABI_VERSION 19

/* Return codes. */
#define NS_OK 0
#define NS_ERR_INVALID 1   /* argument validation failed; nothing was launched */
#define NS_ERR_LAUNCH 2    /* the HIP runtime rejected a launch */

/* CSR weight encodings (reference: csrc/compartmental.cu:92-119). */
#define NS_WEIGHT_F32 0    /* float32[M] */
#define NS_WEIGHT_F16 1    /* IEEE binary16[M] */
#define NS_WEIGHT_E4M3 2   /* OCP fp8 e4m3fn codes uint8[M] x float32 global scale */
#define NS_WEIGHT_NVFP4 3  /* e2m1 nibbles uint8[ceil(M/2)] (even edge in the low nibble),
                              e4m3fn block scales uint8[ceil(M/16)] (16 edges per block, in
                              CSR order), float32 global scale */

/* A [B,N] float32 operand read as data[b*stride_b + n*stride_n].  A NULL
 * `data` means every element equals `scalar` (the reference's
 * `input=None, input_scalar=x` convention, compartmental.cu:41-45). */
typedef struct ns_plane {
  const float* data;
  int64_t stride_b;
  int64_t stride_n;
  float scalar;
} ns_plane;

/* A [B,N] float32 output written as data[b*stride_b + n*stride_n]. */
typedef struct ns_out_plane {
  float* data;
  int64_t stride_b;
  int64_t stride_n;
} ns_out_plane;

/* An [N] float32 vector read as data[n*stride]; stride 0 broadcasts one value. */
typedef struct ns_vector {
  const float* data;
  int64_t stride;
} ns_vector;

/* Destination-major CSR matrix W[N,N] (row = target neuron, col = source). */
typedef struct ns_csr {
  int64_t n_rows;              /* N */
  int64_t n_edges;             /* M */
  const int32_t* rowptr;       /* [N+1], rowptr[0] = 0, rowptr[N] = M, non-decreasing */
  const int32_t* col;          /* [M], each in [0, N) */
  const void* weight;          /* encoding given by `format` */
  int32_t format;              /* NS_WEIGHT_* */
  const uint8_t* block_scales; /* NVFP4 only, else NULL */
  const float* global_scale;   /* device float32[1]; E4M3/NVFP4 only, else NULL */
} ns_csr;

/* Row blocks produced by ns_plan_row_blocks and copied to the device:
 * `bounds` holds (row, edge) int32 pairs for block boundaries 0..n_blocks,
 * bounds[2k] = first row of block k, bounds[2k+1] = rowptr[that row]. */
typedef struct ns_row_plan {
  const int32_t* bounds;       /* device int32[2*(n_blocks+1)] */
  int64_t n_blocks;
  int32_t block_edges;         /* edges per block the plan was built for (<= ns_block_edges) */
  int32_t reserved;
} ns_row_plan;

/* Column-panel layout of a CSR matrix for batch widths 1 and 2, built by
 * ns_plan_panels.  Columns are cut into `n_panels` panels of `panel_width`
 * neurons (a panel's slice of the state fits in one workgroup's LDS).  Rows
 * are cut into `n_ranges` ranges shared by every panel.  A tile is one
 * workgroup's work: one panel and one row range.  The
 * tile's rows are sorted by the length of their segment in the panel and cut
 * into groups; a group gives each of its rows 2^lg lanes of a 64-lane
 * wavefront (64 >> lg rows), lane j of a row taking the row's edges j, j+2^lg,
 * ...  Every group has at least one step.  A group's slots are step-major:
 * slot (step k, lane l) is first_slot + 64*k + l.  Each of the tile's `waves`
 * wavefronts owns a run of consecutive groups whose slots are contiguous (its
 * stream).  Padding slots have source index `panel_width` (a zero kept in LDS)
 * and weight code 0.  Edge slot k is original CSR edge perm[k] (or padding). */
/* Panel layout flag: pair layout.  Every row gets at least two lanes, and
 * within each (row, panel) segment the edges are grouped by 16-edge weight
 * block (stable) with each block's run padded to an even length.  Slots 2i and
 * 2i+1 then hold edges of one block (or padding), and NVFP4 weights take one
 * uint16 word per slot pair: the two nibbles in the low byte (slot 2i in the
 * low nibble) and the pair's e4m3 block-scale code in the high byte. */
#define NS_PANEL_PAIRS 1

/* Panel plan flag (set by the caller, not the planner): finish the tick with a
 * second launch that adds each row's panel sums and applies the update,
 * instead of letting the last tile of each row range do it in the same launch.
 * The results are bitwise the same. */
#define NS_PANEL_COMBINE_LAUNCH 2
/* ns_panel_plan flag: `weight` holds each slot's CSR edge number (int32, -1 for
 * padding: the plan's perm) instead of its weight, and the tick reads the
 * float32 weight of that edge from the matrix's CSR-order weights
 * (NS_WEIGHT_F32 only).  Ticks on a weight version used once then need no
 * slot-order copy (ns_gather_slot_weights). */
#define NS_PANEL_INDEXED 4

typedef struct ns_panel_plan {
  int32_t panel_width;
  int32_t n_panels;
  int32_t n_tiles;
  int32_t n_groups;
  int32_t waves;               /* wavefronts per workgroup the plan was built for */
  int32_t flags;               /* NS_PANEL_* flags */
  int32_t n_ranges;            /* row ranges; each panel has one tile per range */
  int32_t reserved;
  int64_t n_slots;             /* edge slots including padding and the tail padding */
  int64_t n_step_words;        /* uint32 words of `last_steps` */
  const int32_t* tiles;        /* [n_tiles][4]: panel, first row, end row, first entry of
                                  the tile's rows in `rows` */
  const int32_t* tile_ranges;  /* [n_tiles]: row range of each tile */
  const int32_t* wave_groups;  /* [n_tiles*waves + 1]: wave w of tile t owns groups
                                  wave_groups[t*waves+w] .. wave_groups[t*waves+w+1]-1 */
  const int32_t* groups;       /* [n_groups][4]: first slot, steps, lg | rows << 8,
                                  first entry in `rows` */
  const uint16_t* rows;        /* tile-local row (row - tile's first row) of each group row */
  const uint32_t* last_steps;  /* bit k set: step k (slots 64k .. 64k+63) is a group's last */
  const uint16_t* col;         /* [n_slots] source index minus the panel's first neuron */
  const void* weight;          /* [n_slots] weights in slot order, encoding of the matrix:
                                  F32/F16 values, E4M3 codes, NVFP4 nibbles (two per byte;
                                  pair layouts: one uint16 word per slot pair, see
                                  NS_PANEL_PAIRS); with NS_PANEL_INDEXED, int32 CSR edge
                                  numbers (-1: padding) */
  const uint8_t* slot_scales;  /* NVFP4 without NS_PANEL_PAIRS: e4m3 block-scale code of
                                  each slot's edge (unused with NS_PANEL_PAIRS) */
  float* partials;             /* workspace float[2][n_panels*N*batch]: the second half
                                  holds row sums in row-table order, the first half the
                                  per-panel row sums by row (several panels), added in
                                  panel order once every panel's tile of the row range
                                  has stored them */
  uint32_t* range_counters;    /* workspace uint32[n_ranges] (several panels, unless
                                  NS_PANEL_COMBINE_LAUNCH): zero before the first launch;
                                  each tile adds one to its range's counter after storing
                                  its sums, and the tile that brings it to n_panels
                                  finishes the range's rows and sets it back to zero, so
                                  every launch leaves the counters zero.  Launches sharing
                                  a plan's workspace must be ordered on one stream. */
} ns_panel_plan;

/* Source-band layout of a CSR matrix for wide batches (batch a multiple of
 * 4, neuron-major state), built by ns_plan_bands.  Sources are cut into
 * `n_bands` bands of `band_width` neurons; a band of the state (band_width x
 * 16, 8 or 4 floats per column tile) is sized to stay resident in one XCD's L2 while
 * every workgroup on that XCD gathers from it.  Destination rows are cut into
 * `n_row_blocks` blocks of `block_rows` rows; one workgroup owns one block
 * (and one tile of 16, 8 or 4 columns), keeps the block's row sums in LDS, walks the
 * bands in order, passing a workgroup barrier after each, and finally applies
 * the update.  Per band, the block's rows with edges in the band are packed
 * into groups of 64 lanes: a group's first rows are the 64 longest segments
 * left (longest first), and the group lasts as many steps as its longest.  A
 * lane takes its first row's segment in CSR order and, in the steps after it,
 * possibly a second row's segment (the longest left that fits, lanes with the
 * most spare steps choosing first).  Each group goes to the one of the
 * NS_BAND_WAVES wavefronts with the fewest steps in the band so far, so a
 * row's groups of different bands may lie in different wavefronts.  A group is
 * cut into register blocks of `block_steps` steps (its last block may count
 * fewer; its slots past that count are padding).  A block's slots are
 * lane-major: slot (lane l, step k) is 64*first_step + l*block_steps + k, so a
 * lane's steps are consecutive.  A wavefront's blocks are consecutive in
 * `blocks`, in band order, and their slots contiguous.
 * Padding slots have source index 0xFFFF and weight code 0.  Slot k is
 * original CSR edge perm[k] (or padding).  The kernel reads one block record
 * and one register block of slots ahead, so the tables end with a sentinel
 * block record (whose group is a last group of 64 padding rows) and 8*64
 * padding slots. */
/* Wavefronts per band workgroup: `wave_blocks` holds NS_BAND_WAVES entries per
 * row block (plus one). */
#define NS_BAND_WAVES 16

typedef struct ns_band_plan {
  int32_t band_width;          /* source neurons per band, at most 65535 */
  int32_t n_bands;
  int32_t block_rows;          /* destination rows per workgroup */
  int32_t n_row_blocks;
  int32_t n_blocks;            /* register blocks over all wavefronts (sentinel excluded) */
  int32_t n_groups;
  int32_t block_steps;         /* steps per register block the plan was cut for */
  int32_t reserved;
  int64_t n_slots;
  const int32_t* wave_blocks;  /* [n_row_blocks*NS_BAND_WAVES + 1]: wavefront w of row
                                  block q owns blocks wave_blocks[NS_BAND_WAVES*q + w] ..
                                  wave_blocks[NS_BAND_WAVES*q + w + 1] - 1 */
  const int32_t* blocks;       /* [n_blocks+1][4]: first step, band,
                                  steps | last << 8 | step in group << 9 (last: the block
                                  ends its group), group */
  const uint32_t* rows;        /* [n_groups][64] lane words: block-local first row (bits
                                  0-11) and second row (bits 12-23), 0xFFF none, and the
                                  step in the group where the second row starts (bits
                                  24-31; 0 without a second row) */
  const uint16_t* col;         /* [n_slots] source index minus the band's first neuron;
                                  16-byte aligned, as are weight and slot_scales */
  const void* weight;          /* [n_slots] weights in slot order, encoding of the matrix */
  const uint8_t* slot_scales;  /* NVFP4: e4m3 block-scale code of each slot's edge */
} ns_band_plan;

/* Arguments of one fused matrix tick. */
typedef struct ns_step_args {
  int64_t n_neurons;           /* N > 0 */
  int64_t batch;               /* B >= 0; B == 0 launches nothing */
  ns_plane state;              /* s_t   (data required) */
  ns_plane dendrite;           /* d_t   (data required) */
  ns_plane adaptation;         /* a_t   (data required) */
  ns_plane drive;              /* somatic drive u        (data or scalar) */
  ns_plane dendritic_drive;    /* dendritic drive v      (data or scalar) */
  ns_vector params[6];         /* alpha, gain, rho_d, rho_a, coupling, strength */
  ns_csr matrix;
  ns_row_plan plan;
  const ns_panel_plan* panels; /* optional (batch <= 2): column-panel layout to use
                                  instead of the row plan; NULL selects the row plan */
  ns_out_plane out_state;      /* s_{t+1}; must not overlap any input */
  ns_out_plane out_dendrite;   /* d_{t+1} */
  ns_out_plane out_adaptation; /* a_{t+1} */
  ns_out_plane out_current;    /* optional: j = W @ s_t as well (data NULL: not written);
                                  a recorded tick keeps it for its backward */
} ns_step_args;

/* Arguments of one PELS event tick (advance + emit, then scatter). */
typedef struct ns_event_args {
  int64_t n_neurons;
  int64_t batch;
  ns_plane state, dendrite, adaptation;
  ns_plane drive, dendritic_drive;
  ns_vector params[6];
  float* current;              /* persistent synaptic current, [B,N] read as
                                  current[b*current_stride_b + n*current_stride_n];
                                  read by the advance, then updated in place */
  int64_t current_stride_b;
  int64_t current_stride_n;
  ns_plane emitted;            /* last emitted somatic state (data required) */
  ns_vector theta;             /* per-neuron emission threshold */
  const int32_t* out_rowptr;   /* source-major CSR: [N+1] */
  const int32_t* dst;          /* [M] target of each source-major edge */
  const int32_t* weight_index; /* [M] position of that edge in `weight` */
  const float* weight;         /* [M] destination-major float32 weights */
  int64_t n_edges;
  ns_out_plane out_state, out_dendrite, out_adaptation, out_emitted;
  float* delta;                /* workspace float32[B*N], overwritten (two-launch tick) */
  /* Optional, both or neither: the one-launch tick.  Each is float32[B*N],
     entry n*B + b.  The true persistent current is then `current` plus the
     pending contributions: on entry the tick reads j = current + pending_in,
     stores j into `current` and zeroes pending_in; the emitters' out-edges are
     added into pending_out, which must be zero on entry.  The caller swaps the
     two buffers between ticks, or adds pending_out into `current` and zeroes
     it.  `delta` is not used.  With NS_EVENT_ADVANCE_ONLY, pending_in alone
     may be given (pending_out NULL): the launch folds it into `current` the
     same way and writes the deltas to `delta`. */
  float* pending_in;
  float* pending_out;
  /* Optional: the weights in source-major order, out_weight[e] ==
     weight[weight_index[e]], so the scatter streams them instead of gathering
     through weight_index (NULL: gather). */
  const float* out_weight;
  int32_t flags;               /* NS_EVENT_* */
  int32_t reserved;
  /* Optional, one-launch forms only (pending_in given): counters of
     int64[NS_EVENT_ACTIVITY_SLOTS * NS_EVENT_ACTIVITY_STRIDE].  The tick adds
     the out-degree of every active (neuron, column) pair, |s' - emitted| >=
     theta, to counter k * NS_EVENT_ACTIVITY_STRIDE for some k below
     NS_EVENT_ACTIVITY_SLOTS; the sum of those counters grows by the tick's
     active out-edges, the reference's PELS policy measure (runtime.py:129-165).
     The caller zeroes and reads them (NULL: not counted). */
  int64_t* activity;
} ns_event_args;

#define NS_EVENT_ACTIVITY_SLOTS 32
#define NS_EVENT_ACTIVITY_STRIDE 16

/* ns_event_args flag: run the advance and emission only (the two-launch
 * tick's first kernel; `delta` required, one-launch buffers not allowed) and
 * leave the propagation of `delta` to the caller, for instance as
 * current += W @ delta with ns_csr_spmm (`accumulate`): the reference's matrix
 * propagation of emitted deltas (runtime.py:233-235), which beats the scatter
 * when many sources emit. */
#define NS_EVENT_ADVANCE_ONLY 1

/* Arguments of a plain CSR product J = W @ S (no neuron update). */
typedef struct ns_spmm_args {
  int64_t n_neurons;
  int64_t batch;
  ns_plane source;             /* S, [B,N] (data required) */
  ns_csr matrix;
  ns_row_plan plan;
  ns_out_plane out;            /* J, [B,N]; must not overlap `source` */
  int32_t accumulate;          /* nonzero: out += W @ S (every (b, n) of `out` a distinct
                                  element) instead of out = W @ S */
  int32_t reserved;
  const ns_panel_plan* panels; /* optional (batch 1 or 2): run the product on this
                                  column-panel layout of the matrix (ns_plan_panels over
                                  the same CSR; slot weights or NS_PANEL_INDEXED, as for
                                  ns_dendritic_step), summed in panel order and added
                                  or stored by the combine kernel; `plan` is then not
                                  read.  NULL: row blocks. */
} ns_spmm_args;

/* Arguments of the backward of one fused matrix tick (float32 weights). */
typedef struct ns_step_grad_args {
  int64_t n_neurons;           /* N > 0 */
  int64_t batch;               /* B >= 0; B == 0 launches nothing */
  ns_plane state;              /* the forward's inputs, as passed to ns_dendritic_step */
  ns_plane dendrite;
  ns_plane adaptation;
  ns_plane drive;
  ns_plane dendritic_drive;
  ns_vector params[6];
  ns_csr matrix;               /* NS_WEIGHT_F32 only */
  ns_row_plan plan;            /* row plan of `matrix` for batch width B */
  const int32_t* out_rowptr;   /* source-major view of the same graph: [N+1] */
  const int32_t* dst;          /* [M] */
  const int32_t* out_weight_index;  /* [M]: canonical edge -> CSR position */
  ns_plane grad_state;         /* upstream gradients of s', d', a'; a NULL plane with */
  ns_plane grad_dendrite;      /* scalar 0 means zero */
  ns_plane grad_adaptation;
  ns_out_plane d_state;        /* required */
  ns_out_plane d_dendrite;     /* required */
  ns_out_plane d_adaptation;   /* required */
  ns_out_plane d_drive;        /* data NULL: not computed */
  ns_out_plane d_dendritic_drive;
  float* d_weight;             /* [M] in CSR order; NULL: not computed */
  float* d_params[6];          /* [N] each, per neuron; NULL: not computed */
  float* workspace;            /* ns_step_backward_workspace_floats(N, B) floats */
  const float* current;        /* optional [N*B]: j = W @ s of the forward, neuron-major
                                  (j[n*B + b]), as ns_dendritic_step's out_current wrote
                                  it; NULL: recomputed from the CSR */
  const float* out_weight;     /* optional [M]: the CSR weights in source-major order,
                                  out_weight[e] == matrix.weight[out_weight_index[e]];
                                  when set, the transposed product streams it instead of
                                  gathering through out_weight_index (NULL: gather) */
  const ns_panel_plan* transposed_panels;  /* optional, batch 1 or 2: a panel plan (built
                                  by ns_plan_panels with batch B) of the transposed
                                  matrix, whose rows are the sources (out_rowptr, dst) and
                                  whose slot weights are matrix.weight in its slot order
                                  (slot k: matrix.weight[out_weight_index[e]] for the
                                  source-major edge e the plan's perm names).  When set,
                                  the transposed product runs the panel kernel's stream
                                  and per-panel sums (then a second kernel adds them into
                                  d_state) instead of the out-edge walk; out_weight is
                                  then unused.  Its partials workspace must not overlap
                                  the gradient planes or the workspace. */
} ns_step_grad_args;

/* Arguments of one weight encoding (fp8 e4m3 or NVFP4 CSR payload). */
typedef struct ns_encode_args {
  const float* weight;         /* [n_edges] float32 in CSR order, 16-byte aligned */
  int64_t n_edges;             /* M >= 0 */
  int32_t format;              /* NS_WEIGHT_E4M3 or NS_WEIGHT_NVFP4 */
  int32_t reserved;
  uint8_t* codes;              /* E4M3: [M] codes (4-byte aligned); NVFP4: [(M+1)/2]
                                  bytes, even edge in the low nibble (8-byte aligned) */
  uint8_t* block_scales;       /* NVFP4: [(M+15)/16] e4m3 codes; E4M3: unused */
  float* global_scale;         /* device float32[1] */
  uint32_t* workspace;         /* ns_encode_workspace_bytes() bytes, contents ignored */
} ns_encode_args;

/* Arguments of one graph build (coalescing and both CSR views) on the device. */
typedef struct ns_topology_args {
  int64_t n_neurons;           /* N in [1, 2^31] */
  int64_t n_candidates;        /* Mc in [0, 2^31): candidate edges, duplicates allowed */
  const int64_t* src;          /* [Mc] device, each in [0, N) (not checked on the device) */
  const int64_t* dst;          /* [Mc] device, each in [0, N) */
  const float* weight;         /* [Mc] device */
  /* Outputs, device, sized for Mc edges; the first *n_edges entries are the graph. */
  int32_t* out_src;            /* [Mc] canonical (src, dst)-ordered sources */
  int32_t* out_dst;            /* [Mc] */
  float* out_weight;           /* [Mc] summed weights */
  int32_t* out_rowptr;         /* [N+1] source-major offsets */
  int32_t* in_rowptr;          /* [N+1] destination-major offsets */
  int32_t* in_col;             /* [Mc] source of each destination-major edge */
  float* in_weight;            /* [Mc] */
  int32_t* out_weight_index;   /* [Mc] canonical edge -> destination-major position */
  int64_t* n_edges;            /* device int64[1]: the coalesced edge count M */
  void* workspace;             /* ns_topology_workspace_bytes(N, Mc) bytes, 256-byte aligned */
  int64_t workspace_bytes;
} ns_topology_args;

/* ABI version of the loaded library (NS_ABI_VERSION). */
int ns_abi_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* ns_last_error(void);

/* Edge capacity of one row block used by the tick kernels for batch width
 * `batch`: a plan passed to ns_dendritic_step/ns_csr_spmm must have been built
 * with at most this many edges per block (a multiple of 4, at least 8).
 * Smaller blocks give small graphs more workgroups. */
int32_t ns_block_edges(int64_t batch);

/* Host-side planner: splits rows [0,N) of a host copy of `rowptr` into blocks
 * of consecutive rows whose edges fit `block_edges` (with the 4-edge alignment
 * slack the kernels use) and at most 256 rows; a row too long for one block
 * gets a block of its own.  Writes 2*(n_blocks+1) int32 into `bounds` when
 * `capacity` (in int32 elements) suffices; always stores the block count in
 * *n_blocks.  Validates rowptr (monotone, rowptr[0] == 0). */
int ns_plan_row_blocks(const int32_t* rowptr_host, int64_t n_rows, int32_t block_edges,
                       int32_t* bounds, int64_t capacity, int64_t* n_blocks);

/* Host-side panel planner for a host copy of (rowptr, col).  Panel width is
 * the largest that fits `max_panel_width` neurons, equalised over panels and
 * rounded to a multiple of 4.  Rows are cut into about `tiles_per_panel`
 * ranges of equal cost over all panels (items + 1 per row and panel, at most
 * 65536 rows each); each panel has one tile per range.  A row whose segment has L edges gets the smallest
 * power-of-two lane count that leaves each lane at most `lane_target` edges
 * (at most 64; at least 2 with NS_PANEL_PAIRS in `flags`, where a segment's
 * length counts its padding items).  Groups go to the `waves` wavefronts of their tile (which
 * must be the kernel's wavefronts per workgroup) longest first onto the
 * least-loaded one.  Call once with all output pointers NULL to get the sizes
 * in *plan (n_panels, panel_width, n_tiles, n_groups, n_slots, waves,
 * n_step_words, n_ranges) and *n_row_entries, then again with arrays of those
 * sizes: tiles int32[4*n_tiles], tile_ranges int32[n_tiles], wave_groups
 * int32[n_tiles*waves+1], groups
 * int32[4*n_groups], rows uint16[n_row_entries], last_steps
 * uint32[n_step_words], perm int32[n_slots] (-1 for padding), col
 * uint16[n_slots].  Pointer fields of *plan are not touched. */
int ns_plan_panels(const int32_t* rowptr_host, const int32_t* col_host, int64_t n_rows,
                   int32_t max_panel_width, int32_t tiles_per_panel, int32_t waves,
                   int32_t lane_target, int32_t flags, ns_panel_plan* plan,
                   int64_t* n_row_entries,
                   int32_t* tiles, int32_t* tile_ranges, int32_t* wave_groups, int32_t* groups,
                   uint16_t* rows, uint32_t* last_steps, int32_t* perm, uint16_t* col);

/* Panel geometry the tick kernels use for batch width `batch` (1 or 2):
 * largest panel width and the wavefronts per workgroup (NULL outputs are
 * skipped). */
int ns_panel_geometry(int64_t batch, int32_t* max_panel_width, int32_t* waves);

/* The weights of a CSR payload (original edge order, format NS_WEIGHT_*)
 * rearranged into a panel or band layout's slot order: slot k holds edge
 * perm[k] (perm[k] < 0 or >= n_edges: padding, code 0), as the `weight` (and
 * `slot_scales`) arrays of ns_panel_plan / ns_band_plan take them.  No
 * counterpart in the reference (whose kernel reads the CSR in place); it is
 * what a layout rebuilds when the weights change.  n_slots even.  Outputs:
 * F32 float[n_slots], F16 uint16[n_slots], E4M3 uint8[n_slots]; NVFP4
 * uint8[n_slots/2] nibbles (slot 2i low) plus slot_scales uint8[n_slots], or,
 * with `pairs`, uint16[n_slots/2] words (nibbles low, the pair's first real
 * edge's block-scale code high) and no slot_scales.  One launch on `stream`. */
int ns_gather_slot_weights(const int32_t* perm, int64_t n_slots, int64_t n_edges,
                           int32_t format, int32_t pairs, const void* weight,
                           const uint8_t* block_scales, void* slots, uint8_t* slot_scales,
                           void* stream);


/* Fused matrix tick.  Replaces dendritic_step
 * (reference: csrc/bindings.cpp:3-7,137-142; csrc/compartmental.cu:176-236),
 * except that the caller supplies the output planes and the row plan. */
int ns_dendritic_step(const ns_step_args* args, void* stream);

/* Host-side band planner for a host copy of (rowptr, col): `band_width`
 * sources per band (1..65535), `block_rows` destination rows per workgroup
 * (1..4095; the tick takes at most ns_band_max_block_rows(batch)), register
 * blocks of at most `block_steps`
 * steps (1..8).  Call once with all output pointers NULL to get the sizes in
 * *plan (n_bands, n_row_blocks, n_blocks, n_groups, n_slots), then again with
 * wave_blocks int32[NS_BAND_WAVES*n_row_blocks+1], blocks int32[4*(n_blocks+1)], rows
 * uint32[64*n_groups], perm int32[n_slots] (-1 for padding), col
 * uint16[n_slots].  Pointer fields of *plan are not touched.  blocks holds
 * n_blocks records plus the sentinel, rows n_groups groups including the
 * sentinel group, and the slots end with 8*64 padding slots. */
int ns_plan_bands(const int32_t* rowptr_host, const int32_t* col_host, int64_t n_rows,
                  int32_t band_width, int32_t block_rows, int32_t block_steps,
                  ns_band_plan* plan, int32_t* wave_blocks, int32_t* blocks, uint32_t* rows,
                  int32_t* perm, uint16_t* col);

/* Largest block_rows the band tick takes at this batch: its LDS holds each
 * row's sums over the workgroup's column tile, 2496 rows of 16 columns, 4095
 * (the lane word's limit) of 8 or 4. */
int32_t ns_band_max_block_rows(int64_t batch);

/* Fused matrix tick over a band layout (batch a multiple of 4, state
 * neuron-major with 16-byte aligned rows; workgroups take 16 state columns
 * when the batch is a multiple of 16, else 8 when it is a multiple of 8, else
 * 4).  Same semantics and arguments as
 * ns_dendritic_step (it replaces the same reference entry,
 * csrc/bindings.cpp:3-7,137-142; csrc/compartmental.cu:176-236); `args->plan`
 * and `args->panels` are ignored, the CSR in `args->matrix` gives only the
 * weight format and global scale, and the slots come from `plan`. */
int ns_dendritic_step_bands(const ns_step_args* args, const ns_band_plan* plan, void* stream);

/* PELS event tick: advance + emission threshold, then scatter of each
 * emitter's out-edges into `current` with float32 atomics.  Replaces
 * dendritic_event (reference: csrc/bindings.cpp:8-12,143;
 * csrc/compartmental.cu:238-273), except that the caller supplies the four
 * output planes and the delta workspace.  The emitted output follows the
 * reference runtime (runtime.py:241-242): emitted + delta.  With pending_in
 * and pending_out set, the tick is one launch and its scatter goes to
 * pending_out instead of `current` (see ns_event_args). */
int ns_dendritic_event(const ns_event_args* args, void* stream);

/* CSR product J = W @ S with the tick's decoding and summation order (row
 * blocks, or column panels when `panels` is set).
 * Replaces MatrixRuntime._propagate (reference: runtime.py:78-79) for device
 * float32 operands, e.g. the persistent current W @ emitted of runtime.py:124,220,
 * and the matrix propagation of emitted deltas (runtime.py:233-235). */
int ns_csr_spmm(const ns_spmm_args* args, void* stream);

/* Floats of workspace ns_dendritic_step_backward needs (2*N*B). */
int64_t ns_step_backward_workspace_floats(int64_t n_neurons, int64_t batch);

/* Gradients of one fused float32 matrix tick: given the forward's inputs and
 * upstream gradients of (s', d', a'), writes the gradients of the three
 * states, of tensor drives, of the six parameter vectors (per neuron) and of
 * the CSR weights.  Replaces autograd through the reference's torch step,
 * which the reference's native runtime falls back to whenever a gradient is
 * needed (reference: src/neurosim_gpu/native_compartmental.py:104-108; the
 * step compartmental.py:152-183 and runtime.py:78-79, the CSR gradients as
 * in compartmental.py:40-56).  No atomics: results are deterministic. */
int ns_dendritic_step_backward(const ns_step_grad_args* args, void* stream);

/* Bytes of the workspace ns_encode_weights needs (independent of M). */
int64_t ns_encode_workspace_bytes(void);

/* Encodes float32 CSR weights into the fp8 (per-tensor scale) or NVFP4
 * (16-edge e4m3 block scales, float32 global scale) payload that
 * ns_dendritic_step decodes, bit-exact with the reference's encoders.
 * Replaces encode_sparse_weights (reference: src/neurosim_gpu/precision.py:76-90,
 * with _encode_e4m3 :45-49 and _encode_e2m1 :52-73) as called on a weight
 * change (native_compartmental.py:114-124).  Two launches on `stream`, no
 * allocation, no host synchronisation; parity is defined for finite weights. */
int ns_encode_weights(const ns_encode_args* args, void* stream);

/* No counterpart in the reference: ns_encode_weights for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid allocation).  Same arguments and bit-identical
 * results, except that `args->workspace` must be NULL: the amax partials go to
 * a library-owned device array of 4 KiB (1024 partials, enough for every
 * n_edges the encoder accepts, [0, 2^40)), one per GPU, held until the process
 * ends.  Its address is looked up on the first call on each device, with that
 * device current; `stream` must belong to the current device.  Nothing in the
 * array needs clearing (each call rewrites every partial it reads), but calls
 * that overlap on one GPU (on different streams) race on it.  Allocates
 * nothing, launches two kernels on `stream`, no host synchronisation. */
int ns_encode_weights_no_alloc(const ns_encode_args* args, void* stream);

/* Bytes of workspace ns_build_topology needs for N neurons and Mc candidates
 * (-1 on invalid sizes, with ns_last_error set). */
int64_t ns_topology_workspace_bytes(int64_t n_neurons, int64_t n_candidates);

/* Coalesces candidate edges (duplicates summed from zero in input order) and
 * builds both CSR views on the device, bitwise equal to the reference's
 * SparseTopology.from_edges on the CPU (reference:
 * src/neurosim_gpu/topology.py:32-115).  Stable radix sorts and one lane per
 * run of equal keys make the sums deterministic (the reference's GPU path
 * sums duplicates with atomics).  Launches on `stream`; the caller reads
 * *n_edges back to trim the outputs.  Indices must lie in [0, N): the caller
 * checks them, as the reference's from_edges does before building. */
int ns_build_topology(const ns_topology_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NEUROSIM_HIP_H */
