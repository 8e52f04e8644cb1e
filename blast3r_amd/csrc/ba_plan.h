// Constants shared by the plan builder (host C++) and the fused kernels (HIP).
#pragma once

#define BA_CHUNK 128          // observation slots per chunk (one slot per lane in the per-observation phases)
#define BA_MAX_LOCAL 16       // images a batch may touch (bit mask in 32 bits, local ids in 8 bits)
#define BA_WAVES 16           // waves per workgroup of the fused Schur kernel (four per SIMD)
#define BA_SLOTS_PER_WAVE 6   // camera-pair accumulators held in registers by one wave
#define BA_MAX_SLOTS (BA_WAVES * BA_SLOTS_PER_WAVE)
#define BA_MAX_CT 64          // tracks per chunk (coverage bit masks in 64 bits)

// plan arrays (all int32)
enum {
    BA_PA_CHUNK_OBS = 0,
    BA_PA_CHUNK_META,
    BA_PA_SLOT_INFO,
    BA_PA_CT_PID,
    BA_PA_CT_FIRST,
    BA_PA_CT_M,
    BA_PA_CT_MASK,
    BA_PA_B_CHUNK_PTR,
    BA_PA_B_IMGS,
    BA_PA_B_NIMGS,
    BA_PA_B_SLOT_PTR,
    BA_PA_SLOT_PAIR,
    BA_PA_SLOT_GPAIR,
    BA_PA_PAIR_I1,
    BA_PA_PAIR_I2,
    BA_PA_PAIR_PTR,
    BA_PA_PAIR_SRC,
    BA_PA_ROW_PTR,
    BA_PA_ROW_ENT,
    BA_PA_IMG_PTR,
    BA_PA_IMG_SRC,
    BA_PA_CHUNK_SLOTS,      // per chunk, BA_MAX_SLOTS slot table words (BA_TAB, below)
    BA_PA_CHUNK_ENT,        // MFMA entries of every chunk, 32 bits each, see below
    BA_PA_CHUNK_EPTR,       // per chunk, and one past the last: first entry, in units of 4 entries (16 bytes)
    BA_PA_B_POS_SLOT,       // per batch, BA_MAX_SLOTS words: the batch slot at Schur-kernel place
                            // wave + BA_WAVES * k, or -1 (places balanced by work)
    BA_PA_SLOT_SRC,         // per chunk slot: its observation, 0 for an empty slot (a gather index)
    BA_PA_S_PID,            // per chunk slot: track id of its observation (0 when empty)
    BA_PA_S_IMG,            // per chunk slot: image of its observation (0 when empty)
    BA_PA_B_ORDER,          // the batches in Schur-kernel dispatch order (estimated cost, decreasing)
    BA_PLAN_NARRAYS
};

// Per-chunk LDS layout of the Schur kernel's observation blocks: slot s holds its V rows (3 x 16
// doubles) at s * BA_BLK and its weighted camera rows J_c at s * BA_BLK + BA_JROW; a zero block of
// 3 x 16 doubles follows the last slot at BA_ZERO.
#define BA_BLK 97           // doubles per observation block: 6 rows x 16 columns + 1 pad (spreads banks)
#define BA_JROW 48          // first J row of a block
#define BA_ZERO (BA_CHUNK * BA_BLK)

// MFMA entry of a camera-pair slot (32 bits): the LDS offsets, in doubles, of its A rows and its B
// rows, A | B << 16: V rows of two observations (an off-diagonal term, or a run's own V on a
// diagonal slot), the J rows of one observation (A = B) on a diagonal slot, or the zero block
// (padding).  Each slot's list is padded to a multiple of 4 entries (one MFMA group); on a diagonal
// slot the J entries come first, padded to whole groups of their own, so that every group is of one
// kind (J groups negate A).  A chunk holds at most BA_LIST_CAP entries.
#define BA_LIST_CAP 1536
// slot table word of a chunk: entry offset | groups << 12 | J groups << 21
#define BA_TAB(off, ng, njg) ((int32_t)(off) | ((int32_t)(ng) << 12) | ((int32_t)(njg) << 21))
#define BA_TAB_OFF(t) ((t) & 0xfff)
#define BA_TAB_NG(t) (((t) >> 12) & 0x1ff)
#define BA_TAB_NJG(t) (((t) >> 21) & 0x3f)

// plan scalars (int64)
enum {
    BA_PS_N_CHUNKS = 0,
    BA_PS_N_BATCHES,
    BA_PS_N_SLOTS,
    BA_PS_N_PAIRS,
    BA_PS_N_CTRACKS,
    BA_PS_L,
    BA_PS_CHUNK,
    BA_PS_MAX_SLOTS_USED,
    BA_PS_MAX_CHUNKS_PER_BATCH,
    BA_PS_N_PAIR_TERMS,
    BA_PLAN_NSCALARS
};

// ---------------------------------------------------------------------------- pair-major plan
// Structure of the pair-major linearize + Schur path (no chunks or batches, so no limit on track
// length, image-level width up to 32 or co-visibility pattern).  A run is the set of observations of
// one track in one image; runs are numbered image by image, by track id within an image.
enum {
    BA_PM_RUN_PTR = 0,      // (n_runs + 1): run r's observations are run_obs[run_ptr[r] .. run_ptr[r + 1])
    BA_PM_RUN_OBS,          // (n_obs): observation ids grouped by run (the identity when an image's rows are pid-sorted)
    BA_PM_RUN_TRK,          // (n_runs): track of run r
    BA_PM_RUN_IMG,          // (n_runs): image of run r
    BA_PM_IMG_RUN_PTR,      // (n_imgs + 1): runs of image i are img_run_ptr[i] .. img_run_ptr[i + 1]
    BA_PM_TRK_RUN_PTR,      // (n_tracks + 1)
    BA_PM_TRK_RUN,          // (n_runs): runs of each track in image order
    BA_PM_TRK_OBS_PTR,      // (n_tracks + 1)
    BA_PM_TRK_OBS,          // (n_obs): observations of each track in image order
    BA_PM_OBS_IMG,          // (n_obs): image of each observation
    BA_PM_PAIR_I1,          // (n_pairs): image pairs (i1 <= i2) ordered by (i1, i2): the diagonal pair of every
    BA_PM_PAIR_I2,          //   image with observations and every co-visible pair
    BA_PM_ROW_PTR,          // (n_imgs + 1) image rows of the pair structure, as the batched plan's
    BA_PM_ROW_ENT,          // (pair << 1) | transposed
    BA_PM_DIAG_PAIR,        // (n_imgs): pair id of (i, i), or -1
    BA_PM_TERM_PTR,         // (n_pairs + 1): terms of off-diagonal pair p (none for a diagonal pair)
    BA_PM_TERM,             // (2 n_terms): (run in i1, run in i2) of one track, per term
    BA_PM_PAIR_SCHED,       // (n_pairs): the order in which k_pm_pairs takes the pairs: by the smallest first
                            //   image and the largest last image of their terms' tracks, then pair id; pairs
                            //   without terms last
    BA_PM_NARRAYS
};
#define BA_PM_SPAN 512        // observations (runs) per wave of the pair-major per-image sums
enum { BA_PMS_N_RUNS = 0, BA_PMS_N_PAIRS, BA_PMS_N_TERMS, BA_PMS_MAX_TERMS, BA_PMS_MAX_TRACK_RUNS, BA_PM_NSCALARS };
