/*
 * qmm_params.h -- the launch parameter block shared by the host runtime and the gfx950
 * kernels of the small-M affine-quantised matmul.  Plain C layout, passed by value as the
 * single kernel argument.
 */
#ifndef DFQ_QMM_PARAMS_H
#define DFQ_QMM_PARAMS_H

#include <stdint.h>

/* x staging: 512 threads (8 waves) of a workgroup stage the M rows of its k-block's x.  Row r
 * goes to the DFQ_STAGE_TPR threads r*TPR .. r*TPR + TPR - 1 (a multiple of gs/8, so that a
 * group's gs/8 16-byte chunks sit in aligned neighbouring lanes), thread r*TPR + j taking
 * chunks j, j + TPR, j + 2 TPR, ... of the row; DFQ_STAGE_ITEMS(mt) chunks a thread at most
 * (mt = 2 for the 9..16-row kernels, whose one k-block of x at K = 5120 needs up to 16). */
#define DFQ_STAGE_THREADS 512
#define DFQ_STAGE_TPR(M, gs) (((DFQ_STAGE_THREADS / (M)) / ((gs) / 8)) * ((gs) / 8))
#ifndef DFQ_STAGE_ITEMS_16
#define DFQ_STAGE_ITEMS_16 16
#endif
#define DFQ_STAGE_ITEMS(mt) ((mt) == 2 ? DFQ_STAGE_ITEMS_16 : 12)

/* Work decomposition of the fast kernel (a "stream-K" split with a deterministic fix-up):
 *
 *  - output features are cut into T column tiles of 16 (the MFMA N dimension);
 *  - K is cut into chunks of CH super-steps (one super-step = the k span that holds exactly
 *    two quantisation groups per lane half, 64..256 elements; a chunk is one super-step or
 *    the 8 groups whose scales one 16-byte load fetches), and the chunks into nkb k-blocks
 *    whose sizes differ by at most one (k-block kb holds chunks [kb*chunks/nkb,
 *    (kb+1)*chunks/nkb); its x slice must fit in LDS);
 *  - the U = T*SS units (tile, chunk) of a k-block of SS chunks are split into Gkb
 *    contiguous ranges whose sizes differ by at most one (the first U % Gkb get one more);
 *    or, in an "aligned" split of two k-blocks, the T tiles are split that way and each
 *    workgroup takes whole tiles, so that every tile has exactly one part per k-block (a
 *    narrow N is the case Gkb = T, one tile per workgroup);
 *  - inside a workgroup the waves take units of its range one at a time from a counter in
 *    LDS (the first ones by wave index), in a rotated order that starts with the tile shared
 *    with the next workgroup and continues with the one shared with the previous, so that
 *    cross-workgroup fix-ups happen early;
 *  - every unit's partial tile goes to a slot of an LDS ring over the take order (a slot is
 *    reused once its generation allows); the wave that completes a tile's
 *    units in this workgroup (an LDS arrival counter) sums the slots in unit order into the
 *    tile's block of an LDS output area, frees the tile's slots and marks the tile done;
 *  - a tile with exactly two parts in the whole split (its units in two workgroups, or in
 *    two k-blocks of an aligned split) is finished while the streaming goes on: the
 *    workgroup's publisher wave exchanges its part with one 64-bit atomic per element (the
 *    second arriver writes y);
 *  - every other tile -- a whole tile for y, or, in "reduce" splits, a part for its
 *    workspace slot, which a second kernel sums in a fixed order -- is written by the
 *    publisher waves as it finishes, or ("burst" splits, where a workgroup holds many tiles)
 *    by all waves at the end of the workgroup, after a barrier, with 16-byte row stores, so
 *    that no output store interleaves with the weight stream.
 */
typedef struct QmmParams {
    const void* x;          /* [M][K] activations, bf16 or fp16                      */
    const uint32_t* w;      /* [N][K*bits/32] packed codes, element 0 in low bits     */
    const void* scales;     /* [N][K/gs] same dtype as x                              */
    const void* biases;     /* [N][K/gs]                                              */
    const void* lbias;      /* [N] optional linear bias (NULL if none)               */
    void* y;                /* [M][N] output, same dtype as x                         */
    float* slots;           /* workspace: per-tile partial sums                       */
    int32_t M, N, K;
    int32_t mt;             /* row tiles of 8 the launch computes (1: M<=8, 2: M<=16) */
    int32_t T;              /* column tiles of 16                                     */
    int32_t chunks;         /* chunks of K                                            */
    int32_t nkb;            /* k-blocks                                               */
    int32_t Gkb;            /* workgroups per k-block                                 */
    int32_t nslot_kb;       /* partial slots per tile per k-block                     */
    int32_t reduce;         /* 1: shared tiles go to slots summed by dfq_qmm_reduce   */
    int32_t aligned;        /* 1: each workgroup's range is whole tiles (of its k-block) */
    int32_t epi;            /* 1: y = silu(gate) * up of a gate|up weight interleaved
                               by 8 rows (y is [M][N/2])                              */
    int32_t lds_row_stride; /* bytes per staged x row in LDS                          */
    int32_t lds_xsum_off;   /* byte offset of the per-group x sums in LDS             */
    int32_t lds_part_off;   /* byte offset of the per-unit partial tiles in LDS       */
    int32_t lds_cnt_off;    /* byte offset of the per-tile arrival counters in LDS    */
    int32_t lds_gen_off;    /* byte offset of the partial slots' generations in LDS   */
    int32_t lds_tout_off;   /* byte offset of the finished tiles' fp32 sums in LDS, one
                               [mt][n][8] block per tile the range touches            */
    int32_t lds_key_off;    /* byte offset of 16 per-row 64-bit greedy-accept keys    */
    int32_t burst;          /* 1: tiles without a pair exchange leave at the end of the
                               workgroup; 0: the publisher waves write them as they finish */
    int32_t umax;           /* most units one workgroup holds                         */
    int32_t ring;           /* partial-tile slots in LDS (a ring over the take order) */
    int32_t xcd8;           /* 1: the launch's workgroups are dealt to eight XCDs
                               round-robin (workgroup b on XCD b % 8: the whole chip)  */
    int32_t xcd_pair;       /* 1 (with xcd8): every shared tile has one part per k-block,
                               from the same range index, and the launch places those
                               workgroups on one XCD (whose L2 performs their exchange) */
    uint32_t w_bytes;       /* size of w in bytes (< 2^31)                            */
    uint32_t s_bytes;       /* size of scales (= size of biases) in bytes             */
    /* greedy-accept mode (am_keys != NULL; splits without a second pass only): every
     * finished output also folds (its rounded value, its column) into its row's 64-bit key,
     * the last workgroup turns the keys into tokens and the accepted run; y may be NULL */
    uint64_t* am_keys;      /* [16][M] keys, one row of M per workgroup group; zero at rest */
    uint32_t* am_count;     /* 17 arrival counters, 32 words apart; zero at rest            */
    const int32_t* am_proposals;  /* [M-1] or NULL                                         */
    int32_t* am_tokens;     /* [M] or NULL                                                  */
    int32_t* am_accepted;   /* [1] or NULL                                                  */
} QmmParams;

/* Parameters of the generic (stock-op stand-in) kernel. */
typedef struct QmmGenericParams {
    const void* x;
    const uint32_t* w;
    const void* scales;
    const void* biases;
    const void* lbias;
    void* y;
    int32_t M, N, K, bits, gs;
    int32_t xdt, sdt, ydt;  /* 0 bf16, 1 fp16, 2 fp32 */
} QmmGenericParams;

/* Parameters of the stock path's few-row GEMV (qmv): one dtype for x, scales, biases and y,
 * at most 4 rows a launch.  Workgroup b owns output rows [b*base + min(b, rem), +base +
 * (b < rem)) of base = N / G, rem = N % G; its waves take groups of rows from an LDS counter. */
typedef struct QmvParams {
    const void* x;          /* [M][K]                                                 */
    const uint32_t* w;      /* [N][K*bits/32]                                         */
    const void* scales;     /* [N][K/gs]                                              */
    const void* biases;     /* [N][K/gs]                                              */
    const void* lbias;      /* [N] or NULL                                            */
    void* y;                /* [M][N]                                                 */
    int32_t M, N, K;
    int32_t G;              /* workgroups                                             */
    int32_t rows_max;       /* most rows one workgroup owns                           */
    int32_t lds_xsum_off;   /* byte offset of the per-chunk x sums [M][K/kpl] fp32    */
    int32_t lds_cnt_off;    /* byte offset of the row-group take counter              */
    int32_t lds_out_off;    /* byte offset of the workgroup's outputs [M][rows_max] fp32 */
} QmvParams;

/* Logits per block of dfq_argmax_accept: 256 threads x DFQ_ACCEPT_CHUNK / 2048 16-byte loads
 * of 8 logits (a multiple of 2048).  Fewer, longer blocks mean fewer arrivals on the one
 * device-wide counter; measured on MI355X over [M, 151936] bf16 logits (us, M = 8 / 12 / 16):
 * 4096 logits a block 8.8 / 11.9 / 13.4, 8192 6.6 / 8.4 / 9.3, 16384 7.0 / 8.0 / 8.6.  The
 * standalone accept serves the LM heads of 10..16 rows (below that it is fused). */
#ifndef DFQ_ACCEPT_CHUNK
#define DFQ_ACCEPT_CHUNK 16384
#endif

#endif
