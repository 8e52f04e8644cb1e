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
    BA_PA_CHUNK_SLOTS,      // per chunk, BA_MAX_SLOTS words: entry offset | padded entry count << 16
    BA_PA_CHUNK_ENT,        // MFMA entries of every chunk, 16 bits each (two per word), see below
    BA_PA_CHUNK_EPTR,       // per chunk: first entry, in units of 8 entries (16 bytes)
    BA_PA_B_POS_SLOT,       // per batch, BA_MAX_SLOTS words: the batch slot at Schur-kernel place
                            // wave + BA_WAVES * k, or -1 (places balanced by work)
    BA_PA_SLOT_SRC,         // per chunk slot: its observation, 0 for an empty slot (a gather index)
    BA_PA_S_PID,            // per chunk slot: track id of its observation (0 when empty)
    BA_PA_S_IMG,            // per chunk slot: image of its observation (0 when empty)
    BA_PA_B_ORDER,          // the batches in Schur-kernel dispatch order (estimated cost, decreasing)
    BA_PLAN_NARRAYS
};

// MFMA entry of a camera-pair slot: A slot (7 bits) | B slot (7 bits) << 7 | kind << 14, where the
// slots index the chunk's observation blocks and kind is BA_ENT_V (the V rows of A and B),
// BA_ENT_J (the J rows of A = B, A negated) or BA_ENT_PAD (the zero block).  Each slot's list is
// padded to a multiple of 4 entries; a chunk holds at most BA_LIST_CAP entries.
enum { BA_ENT_V = 0, BA_ENT_J = 1, BA_ENT_PAD = 2 };
#define BA_LIST_CAP 1536

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
    BA_PM_NARRAYS
};
#define BA_PM_SPAN 512        // observations (runs) per wave of the pair-major per-image sums
enum { BA_PMS_N_RUNS = 0, BA_PMS_N_PAIRS, BA_PMS_N_TERMS, BA_PMS_MAX_TERMS, BA_PMS_MAX_TRACK_RUNS, BA_PM_NSCALARS };
