// Tile geometry and load / barrier schedule of the halo conv (k_conv3.hip),
// as plain constexpr C++ so that a host program can check the schedule
// (tests/conv3_schedule_check.cpp simulates it for every tile width and
// chunk count against in-order load completion).
#pragma once

namespace di {
namespace conv3 {

constexpr int CV_BM = 128, CV_BN = 64, CV_NT = 512;
constexpr int CV_ROW = 128;              // bytes per LDS row (64 fp16 channels)
constexpr int CV_BBUF = CV_BN * CV_ROW;  // one weight stage: 8 KB
constexpr int CV_LDC = CV_BN + 4;        // fp32 C tile row stride

// Iteration s of a workgroup (stage s = chunk * 9 + tap of its split) reads
// the MFMA fragments of stage s + 1 at its top, runs the MFMAs of stage s,
// issues the weights of stage s + NBB - 1 and, at taps 0..last_tap, the
// patch pieces of the next chunk; a barrier follows every BAR-th iteration,
// before which each wave waits until at most allow(j) of its loads are
// outstanding (loads retire in order) and for its LDS reads.  Stages are
// run in rounds of 18 (two chunks) with round-relative iteration j, then a
// tail chunk of 9 when the split has an odd chunk count.
template <int W>
struct ConvGeo {
  static constexpr int R = CV_BM / W;        // output rows per tile
  static constexpr int PW = W + 2;           // patch width
  static constexpr int PR = (R + 2) * PW;    // patch rows (pixels)
  static constexpr int NP = (PR + 63) / 64;  // patch pieces: one 8-row DMA per wave each
  static constexpr int PROWS = NP * 64;      // patch rows allocated
  // pieces per tap: one at taps 0..NP-1, or two at taps 0..3 when NP > 5
  static constexpr int PPT = NP > 5 ? 2 : 1;
  static constexpr int last_tap = (NP - 1) / PPT;  // tap issuing the last piece
  // weight stage buffers (weights issued five iterations ahead) and barrier
  // cadence: a barrier after every second iteration, i.e. per 16 MFMAs of a
  // wave (a barrier and its waits cost ~140 cycles against 256 of MFMA per
  // SIMD and stage).  Measured on the U-Net step: nine buffers (more slack
  // for weights streaming from HBM, 141 KB of LDS at W = 64) cost 1 %
  static constexpr int NBB = 6;
  static constexpr int BAR = 2;
  static_assert(18 % NBB == 0 && 18 % BAR == 0 && BAR <= 2 && NBB >= 5, "static indices over a round");
  // the prologue issues the first chunk's patch and the weights of stages
  // 0..NBB-2, then waits for the patch and stages 0..2 (read before the
  // first barrier) and leaves stages 3..NBB-2 in flight: the first round's
  // iteration -m stands for the load of stage NBB-1-m
  static constexpr int prologue_allow = NBB - 4;
  static constexpr int SMEM_PIPE = 2 * PROWS * CV_ROW + NBB * CV_BBUF;
  static constexpr int SMEM_C = 2 * CV_BM * CV_LDC * 4;  // the two k halves' fp32 tiles
  static constexpr int SMEM = SMEM_PIPE > SMEM_C ? SMEM_PIPE : SMEM_C;
  static_assert(NP <= 8 && last_tap <= 4, "patch pieces issued by tap 4");
  static_assert(SMEM <= 160 * 1024, "LDS");

  // patch pieces issued at tap t
  static constexpr int pieces(int t) {
    return t * PPT >= NP ? 0 : (NP - t * PPT < PPT ? NP - t * PPT : PPT);
  }
  // vector-memory loads of round iteration i (one weight stage plus the
  // pieces of its tap); negative i: the previous round's iteration 18 + i
  static constexpr int issued(int i) { return 1 + pieces(((i % 9) + 9) % 9); }
  // the barrier after round iteration j must have completed every load of
  // iterations <= complete_through(j): the weights of the stages the next
  // BAR iterations read (up to j + BAR + 1, issued NBB - 1 iterations
  // earlier) and, when one of those stages starts a chunk, that chunk's
  // patch (issued at taps 0..last_tap of the chunk before)
  static constexpr int complete_through(int j) {
    int x = j + BAR + 2 - NBB;
    for (int t = j + 2; t <= j + BAR + 1; t++)
      if (t % 9 == 0 && t - 9 + last_tap > x) x = t - 9 + last_tap;
    return x;
  }
  // loads that may stay outstanding there (negative iterations: the
  // previous round's, or in the first round the prologue's loads still in
  // flight, one weight stage each)
  static constexpr int allow(int j) {
    int n = 0;
    for (int i = complete_through(j) + 1; i <= j; i++) n += issued(i);
    return n;
  }
  // tail chunk: iteration i issues the weights of its stage i + NBB - 1
  // while that lies in the chunk, and no patch
  static constexpr int tail_issued(int i) { return i < 0 ? issued(i) : (i + NBB - 1 < 9 ? 1 : 0); }
  static constexpr int tail_allow(int j) {
    int n = 0;
    for (int i = j + BAR + 3 - NBB; i <= j; i++) n += tail_issued(i);
    return n;
  }
};

}  // namespace conv3
}  // namespace di
