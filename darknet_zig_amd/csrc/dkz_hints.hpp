// dkz_hints.hpp -- which operands of each op stream past the caches.
//
// A nontemporal (NT) access keeps a line out of the caches' normal
// replacement order. Measured on MI355X, NT loads and stores make every op
// faster when its operands are cold in HBM (a 2-read/1-write stream: 5.5 ->
// 6.5 TB/s), and also in two of the three op sequences of the benchmark's
// configs -- the SGD step (axpy, axpy, scal over 2 x 100 MB: 6.27 -> 6.48 TB/s)
// and the batch-norm forward + leaky sequence (4.09 -> 4.46 TB/s). The
// exception is the batch-norm backward sequence: all seven ops read the same
// delta, which then stays in the 256 MB Infinity Cache between them, so delta
// and the ops that only touch delta keep ordinary accesses (an NT scale_bias
// there costs mean_delta 18 -> 26 us), and only the operands the sequence
// reads once (the activation output y, x_norm, x in variance_delta) are NT.
//
// Bit i of an op's mask marks its operand i; the operand order of each mask is
// given beside it. Every mask can be overridden at build time (-D...).
#pragma once

// elementwise.hip: bit k = input stream k (load), bit 4 = the outputs (store)
#ifndef DKZ_HINT_FILL
#define DKZ_HINT_FILL 0          // out: delta zeroed before accumulation, or a GEMM output
#endif
#ifndef DKZ_HINT_COPY
#define DKZ_HINT_COPY 16         // x (live), y (a backup read in the backward pass): NT store
#endif
// Copies of fewer than DKZ_COPY_SMALL_BYTES (of x) read x nontemporally too:
// measured on MI355X, config 1's copy of 16.8 MB 7.57 -> 7.15 us with the
// layer sequence that re-reads x next unchanged (54.9 -> 54.6 us), while a
// copy of 32.8 MB went 11.9 -> 12.3 us.
#ifndef DKZ_HINT_COPY_SMALL
#define DKZ_HINT_COPY_SMALL 17
#endif
#ifndef DKZ_COPY_SMALL_BYTES
#define DKZ_COPY_SMALL_BYTES (24ull << 20)
#endif
#ifndef DKZ_HINT_AXPY
#define DKZ_HINT_AXPY 19         // x, y loads; y store
#endif
#ifndef DKZ_HINT_SCAL
#define DKZ_HINT_SCAL 17         // x load and store
#endif
#ifndef DKZ_HINT_MUL
#define DKZ_HINT_MUL 0           // x, y
#endif
#ifndef DKZ_HINT_CONSTRAIN
#define DKZ_HINT_CONSTRAIN 0     // x
#endif
#ifndef DKZ_HINT_ACTIVATE
#define DKZ_HINT_ACTIVATE 17     // x load and store
#endif
#ifndef DKZ_HINT_GRADIENT
#define DKZ_HINT_GRADIENT 17     // y (read once) and the delta store; the delta load stays cached
#endif
#ifndef DKZ_HINT_ADD_SCALAR
#define DKZ_HINT_ADD_SCALAR 0    // x (the truth buffer, read next by the cost op)
#endif
#ifndef DKZ_HINT_RAND_UNIFORM
#define DKZ_HINT_RAND_UNIFORM 0  // out: read at once by dropout, again in the backward pass
#endif
#ifndef DKZ_HINT_DROPOUT
#define DKZ_HINT_DROPOUT 0       // x (read next by the following layer), rand
#endif
// Dropout over arrays of DKZ_DROPOUT_LARGE_BYTES and more (its two arrays
// then exceed the 256 MB Infinity Cache, so neither is still there for the
// next reader) reads and writes nontemporally: measured on MI355X at
// [256,512,28,28] (411 MB an array), 217.5-218.8 -> 195.3-196.3 us; NT loads
// alone or the NT store alone changed nothing (219.7-223.1).
#ifndef DKZ_HINT_DROPOUT_LARGE
#define DKZ_HINT_DROPOUT_LARGE 19
#endif
#ifndef DKZ_DROPOUT_LARGE_BYTES
#define DKZ_DROPOUT_LARGE_BYTES (128ull << 20)
#endif
#ifndef DKZ_HINT_ADAM
#define DKZ_HINT_ADAM 31         // w, d, m, v: each read and written once per step
#endif
// pred, truth loads; delta, err stores: all nontemporal. Measured on MI355X
// for softmax_x_ent: [256,1000] 3.30 -> 2.90 us (the layer's two calls 6.84
// -> 6.35), [8192,1000] 25.0 -> 22.9 us (0.66 -> 0.72 of 8 TB/s); loads or
// stores alone gained a third of that.
#ifndef DKZ_HINT_LOSS
#define DKZ_HINT_LOSS 19
#endif

// broadcast.hip: bit 0 = io load, bit 1 = io store, bit 2 = the read-only operand
#ifndef DKZ_HINT_ADD_BIAS
#define DKZ_HINT_ADD_BIAS 3
#endif
// Also runs on delta inside the backward sequence, where the ops after it
// re-read delta: the store stays cached. The load is nontemporal: measured on
// MI355X at config 2's shape, scale_bias alone 38.7 -> 33.9 us (0.66 -> 0.76
// of 8 TB/s) for a backward chain 0.5% slower (6692 -> 6660 GB/s); a
// nontemporal store instead changed neither.
#ifndef DKZ_HINT_SCALE_BIAS
#define DKZ_HINT_SCALE_BIAS 1
#endif
// ... below this many bytes the tensor is a forward activation small enough
// that the ops after it find it again whatever the hint (the backward
// sequence's delta, which must stay cached, is larger at the configs' shapes)
#ifndef DKZ_HINT_SCALE_BIAS_SMALL
#define DKZ_HINT_SCALE_BIAS_SMALL 3
#endif
#ifndef DKZ_SCALE_BIAS_SMALL_BYTES
#define DKZ_SCALE_BIAS_SMALL_BYTES (64ull << 20)
#endif
#ifndef DKZ_HINT_NORMALIZE
#define DKZ_HINT_NORMALIZE 3
#endif
#ifndef DKZ_HINT_NORMALIZE_DELTA
#define DKZ_HINT_NORMALIZE_DELTA 4  // x (its last read); delta stays cached
#endif
#ifndef DKZ_HINT_AVGPOOL_BWD
#define DKZ_HINT_AVGPOOL_BWD 3
#endif

// reduce.hip: bit 0 = first stream, bit 1 = second stream
#ifndef DKZ_HINT_MEAN
#define DKZ_HINT_MEAN 1            // x
#endif
#ifndef DKZ_HINT_VARIANCE
#define DKZ_HINT_VARIANCE 1        // x
#endif
// mean_delta and backward_bias read one tensor, delta, which in the layer's
// backward step the op just before wrote (gradient_array, scale_bias):
// then ordinary loads, which find it in the Infinity Cache and leave it
// there for the ops after (nontemporal loads here cost the config-2 backward
// chain 3.7%). Otherwise (recently_written false) nontemporal loads, which
// stream cold data faster: measured on MI355X at config 2's shape, 18.6 ->
// 17.7 us (0.69 -> 0.73 of 8 TB/s).
#ifndef DKZ_HINT_MEAN_DELTA
#define DKZ_HINT_MEAN_DELTA 0      // delta, just written
#endif
#ifndef DKZ_HINT_MEAN_DELTA_COLD
#define DKZ_HINT_MEAN_DELTA_COLD 1 // delta, not written recently
#endif
#ifndef DKZ_HINT_VARIANCE_DELTA
#define DKZ_HINT_VARIANCE_DELTA 2  // x; delta stays cached
#endif
#ifndef DKZ_HINT_BACKWARD_BIAS
#define DKZ_HINT_BACKWARD_BIAS 0   // delta, just written
#endif
#ifndef DKZ_HINT_BACKWARD_BIAS_COLD
#define DKZ_HINT_BACKWARD_BIAS_COLD 1  // delta, not written recently
#endif
#ifndef DKZ_HINT_BACKWARD_SCALE
#define DKZ_HINT_BACKWARD_SCALE 2  // x_norm (read once); delta stays cached
#endif
#ifndef DKZ_HINT_AVGPOOL_FWD
#define DKZ_HINT_AVGPOOL_FWD 1     // input, read once
#endif

// softmax.hip (contiguous groups): bit 0 = input load, bit 1 = probability
// store, bit 2 = truth load, bit 3 = delta and loss stores; _XENT for the
// softmax layer's fused pass. Measured cold on MI355X (>= 512 MB cycled):
// softmax [8192,1000] 14.9 us cached, 14.0 NT loads, 13.5 NT loads and
// stores, 12.8 NT stores ([256,1000] 3.56 / 3.24 / 3.28 / 3.33 us); the
// fused layer pass [8192,1000] 33.9 -> 26.7 us and [256,1000] 4.4 -> 3.8 us
// with its three outputs stored NT (they are read once, by the cost sum and
// the backward pass).
#ifndef DKZ_HINT_SOFTMAX
#define DKZ_HINT_SOFTMAX 2
#endif
// The fused layer pass also reads the logits and the truth nontemporally
// (each read once): [256,1000] 4.06 -> 3.82 us; the plain softmax keeps its
// cached input load ([8192,1000] 12.6 against 12.8-13.0 us with it NT).
#ifndef DKZ_HINT_SOFTMAX_XENT
#define DKZ_HINT_SOFTMAX_XENT 15
#endif
// pooling.hip forward: bit 0 = input load, bit 1 = output store, bit 2 = index store
// Measured cold at config 5 ([256,512,28,28]), forward / backward us: masks
// 0 / 1 104.0-105.0 / 180.1-181.3; forward 1: 112.3-112.9, 7: 106.9, 6 (NT
// output and index stores): 101.1-101.3, kept off because the next layer
// reads the output at once and may find it in the Infinity Cache; backward
// 3: 216.7-219.5, 7: 196.0-196.1, 5: 180.1-180.4.
#ifndef DKZ_HINT_MAXPOOL_FWD
#define DKZ_HINT_MAXPOOL_FWD 0
#endif
// pooling.hip backward: bit 0 = delta and index loads, bit 1 = prev load, bit 2 = prev store
#ifndef DKZ_HINT_MAXPOOL_BWD
#define DKZ_HINT_MAXPOOL_BWD 1
#endif
// The 3x3 stride-2 kernels' masks (same bits). Their backward lanes read
// overlapping candidate outputs, which the caches share between them: at
// [64,128,56,56] cold, backward masks 1 / 5 (NT delta and index loads)
// 58.7-59.6 us, 0 54.6-54.9, 4 (NT prev store only) 54.3-54.4; forward 0
// 30.9-31.2, 6 30.3-30.4, 1 / 7 48.7-49.2.
#ifndef DKZ_HINT_MAXPOOL3_FWD
#define DKZ_HINT_MAXPOOL3_FWD 0
#endif
#ifndef DKZ_HINT_MAXPOOL3_BWD
#define DKZ_HINT_MAXPOOL3_BWD 4
#endif
// shortcut.hip: bit 0 = add load, bit 1 = out load, bit 2 = out store.
// Measured cold at config 4, us: 1 13.7-13.8, 5 13.5-13.8, 7 13.5-13.6, 3
// 14.1, 0 15.7, 4 15.5.
#ifndef DKZ_HINT_SHORTCUT
#define DKZ_HINT_SHORTCUT 1
#endif

// im2col.hip: bit 1 = column buffer store. Nontemporal although the GEMM
// reads the buffer next: im2col of a [128,56,56] image 8.1 -> 6.6 us, and the
// im2col + GEMM pair of a convolution's forward step no slower (31.9 -> 31.1 us).
#ifndef DKZ_HINT_IM2COL
#define DKZ_HINT_IM2COL 2
#endif

// batchnorm.hip, the fused layer passes. The statistics pass keeps its input
// cached for the apply pass that re-reads it (at config 1 all of it fits the
// Infinity Cache). The backward sums pass reads y and x cached -- two of the
// three inputs the apply pass re-reads, 206 MB, within the 256 MB Infinity
// Cache -- and delta and x_norm nontemporally; the apply pass streams. At
// config 2 (graph replay, cold): 134.5 us with every sums load nontemporal,
// 126.7 with y and x cached; y, delta and x cached 128.7, one of them 128.3-
// 129.3, all four 137-146; walking the apply tiles backwards gained nothing, and
// cached apply loads lost (137-158 us).
// forward statistics: bit 0 = input load
#ifndef DKZ_HINT_BN_STATS
#define DKZ_HINT_BN_STATS 0
#endif
// forward apply: bit 0 = input load, bit 1 = x store, bit 2 = x_norm store,
// bit 3 = output store (x and x_norm are next read by the backward pass; the
// output by the next layer)
#ifndef DKZ_HINT_BN_FWD_APPLY
#define DKZ_HINT_BN_FWD_APPLY 7
#endif
// one-launch backward: bits 0-3 = y, delta, x_norm, x loads, bit 4 = delta
// store (all nontemporal: config 1's shape 28.7 us with delta cached, 22.9
// all NT, against 27.8 for the two passes). The register- and LDS-holding
// variant (config 2) takes bit 4 only: its loads are nontemporal except the
// first read of the part it reads twice, which stays cached for the second.
#ifndef DKZ_HINT_BN_BWD_COOP
#define DKZ_HINT_BN_BWD_COOP 31
#endif
// one-launch forward: the same bits as the apply pass. Measured (graph
// replay, cold; config 1 / config 2's shape): 7 15.3 / 72.3 us; the output
// nontemporal too (15) 14.9 / 71.3, kept cached for the next layer, which
// reads it; 3 16.7 / 72.2, 1 and 5 17.2 / 72.8, 6 17.3 / 78.2, 0 19.4 / 87.3.
#ifndef DKZ_HINT_BN_FWD_COOP
#define DKZ_HINT_BN_FWD_COOP DKZ_HINT_BN_FWD_APPLY
#endif
// backward sums: bit 0 = y, bit 1 = delta, bit 2 = x_norm, bit 3 = x loads
#ifndef DKZ_HINT_BN_BWD_SUMS
#define DKZ_HINT_BN_BWD_SUMS 6
#endif
// backward apply: bit 0 = y, bit 1 = delta, bit 2 = x loads, bit 3 = delta store
// (all nontemporal: 135 us per config-2 step against 139 us with a cached
// delta store)
#ifndef DKZ_HINT_BN_BWD_APPLY
#define DKZ_HINT_BN_BWD_APPLY 15
#endif
