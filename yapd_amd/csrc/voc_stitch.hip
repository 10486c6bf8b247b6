// Chunk stitching of the streaming vocoder (server/vocoder.py:284-320), for a
// whole micro-batch in one launch.
//
// Every job of a batch is one request's chunk: a run of samples of one row of
// the batch's waveform, of which the first samples are blended with the tail
// the request's previous chunk withheld (tail * fade_out + sample * fade_in),
// or, for a first chunk, multiplied by the trim fade; optional zeros go in
// front (pre-roll); the last `fade` samples are withheld as the next tail
// (fp32, before clipping) unless the chunk is final; the rest becomes 16-bit
// PCM: clip to [-1, 1], times 32767, truncated toward zero.  The host works
// out each job's geometry; the kernel does the per-sample arithmetic, with
// every product and sum rounded on its own (the file is built with
// -ffp-contract=off: no fused multiply-add), so the result equals the float32
// numpy expressions of the reference bit for bit.
//
// Grid: y = job, x strides over the job's samples.  Every job is checked
// against the buffers it names and skipped (nothing written) if it does not
// fit, so a bad job table cannot fault.
#include "common.h"
#include "../../include/yapd_vocoder.h"

namespace yapd {
namespace {

constexpr int kStitchThreads = 256;
constexpr int kStitchGridX = 64;

struct StitchParams {
  const float* wav;
  int64_t wav_stride;
  int64_t wav_cols;
  int rows;
  const int32_t* jobs;  // [n_jobs][YAPD_STITCH_JOB_INTS]
  const float* fade_in;
  const float* fade_out;
  int fade;
  const float* trim;
  int n_trim;
  const float* tails_in;  // [n_tails_in][fade]
  int n_tails_in;
  float* tails_out;  // [n_tails_out][fade]
  int n_tails_out;
  int16_t* pcm;
  int64_t pcm_len;
};

__device__ __forceinline__ int16_t to_pcm16(float v) {
  // np.clip(v, -1, 1) * 32767 then astype(int16): truncation toward zero.  A
  // NaN sample becomes the clip's lower bound (-32767).
  const float c = fminf(fmaxf(v, -1.f), 1.f);
  return static_cast<int16_t>(static_cast<int>(c * 32767.f));
}

__global__ __launch_bounds__(kStitchThreads) void voc_stitch_kernel(const StitchParams p) {
  const int32_t* j = p.jobs + static_cast<int64_t>(blockIdx.y) * YAPD_STITCH_JOB_INTS;
  const int row = j[0], lo = j[1], n_seg = j[2], n_blend = j[3], trim = j[4], pre = j[5], n_out = j[6];
  const int tin = j[7], tout = j[8];
  const int64_t pcm_off = static_cast<int64_t>(j[9]);
  const int64_t n_all = static_cast<int64_t>(pre) + n_seg;
  const bool ok = row >= 0 && row < p.rows && lo >= 0 && n_seg >= 0 && pre >= 0 &&
                  static_cast<int64_t>(lo) + n_seg <= p.wav_cols && n_out >= 0 && n_out <= n_all &&
                  pcm_off >= 0 && pcm_off + n_out <= p.pcm_len && n_blend >= 0 && n_blend <= n_seg &&
                  (n_blend == 0 || (tin >= 0 && tin < p.n_tails_in && n_blend <= p.fade)) &&
                  (n_out == n_all || (tout >= 0 && tout < p.n_tails_out && n_all - n_out == p.fade));
  if (!ok) return;
  const float* w = p.wav + static_cast<int64_t>(row) * p.wav_stride + lo;
  const float* tail = p.tails_in + static_cast<int64_t>(tin > 0 ? tin : 0) * p.fade;
  float* tail_out = p.tails_out + static_cast<int64_t>(tout > 0 ? tout : 0) * p.fade;
  const int n_trim = trim ? p.n_trim : 0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kStitchThreads + threadIdx.x; i < n_all;
       i += static_cast<int64_t>(gridDim.x) * kStitchThreads) {
    float v = 0.f;
    if (i >= pre) {
      const int64_t s = i - pre;
      v = w[s];
      if (s < n_trim) v = v * p.trim[s];
      if (s < n_blend) v = tail[s] * p.fade_out[s] + v * p.fade_in[s];
    }
    if (i < n_out) {
      p.pcm[pcm_off + i] = to_pcm16(v);
    } else {
      tail_out[i - n_out] = v;
    }
  }
}

}  // namespace
}  // namespace yapd

extern "C" int yapd_voc_stitch(const float* wav, int64_t wav_stride, int64_t wav_cols, int rows, const int32_t* jobs,
                               int n_jobs, const float* fade_in, const float* fade_out, int fade, const float* trim,
                               int n_trim, const float* tails_in, int n_tails_in, float* tails_out, int n_tails_out,
                               int16_t* pcm, int64_t pcm_len, void* stream) {
  YAPD_REQUIRE(n_jobs >= 0 && n_jobs <= 65535, "voc_stitch: n_jobs must be in [0, 65535] (got %d)", n_jobs);
  if (n_jobs == 0) return YAPD_OK;
  YAPD_REQUIRE(wav && jobs && pcm, "voc_stitch: NULL wav, jobs or pcm");
  YAPD_REQUIRE(rows >= 1 && wav_cols >= 0 && wav_stride >= wav_cols, "voc_stitch: bad wav shape");
  YAPD_REQUIRE(fade >= 1 && fade_in && fade_out, "voc_stitch: need fade >= 1 and both fade ramps");
  YAPD_REQUIRE(n_trim >= 0 && (n_trim == 0 || trim), "voc_stitch: NULL trim");
  YAPD_REQUIRE(n_tails_in >= 0 && (n_tails_in == 0 || tails_in), "voc_stitch: NULL tails_in");
  YAPD_REQUIRE(n_tails_out >= 0 && (n_tails_out == 0 || tails_out), "voc_stitch: NULL tails_out");
  YAPD_REQUIRE(pcm_len >= 0, "voc_stitch: pcm_len must be >= 0");
  yapd::StitchParams p{wav,      wav_stride, wav_cols, rows,       jobs,      fade_in,     fade_out, fade,
                       trim,     n_trim,     tails_in, n_tails_in, tails_out, n_tails_out, pcm,      pcm_len};
  hipLaunchKernelGGL(yapd::voc_stitch_kernel, dim3(yapd::kStitchGridX, static_cast<unsigned>(n_jobs)),
                     dim3(yapd::kStitchThreads), 0, static_cast<hipStream_t>(stream), p);
  YAPD_LAUNCH_CHECK("voc_stitch launch");
  return YAPD_OK;
}
