// Launch of the MFMA decode kernel: picks the variant (per-token K or not, head_dim,
// widest code of the launch, four or eight waves, wave-private group path only or not)
// and sizes its LDS.  The kernel itself is pk_decode_mfma.h, one variant per
// pk_decode_mfma[_tok][_w8|_wo]_<HD>_<MAXB>.hip.
#include "pk_decode_mfma.h"

#include <algorithm>

namespace pk {

static int kivi_group_bytes(int hd, int kb, int vb) {
  return hd == 128 ? kivi_group_bytes_hd<128>(kb, vb) : kivi_group_bytes_hd<64>(kb, vb);
}

static int kivi_stage_bytes(int hd, int kb, int vb) {
  return hd == 128 ? kivi_stage_bytes_hd<128>(kb, vb) : kivi_stage_bytes_hd<64>(kb, vb);
}

static int tok_group_bytes(int hd, int kb, int vb) {
  return hd == 128 ? tok_group_bytes_hd<128>(kb, vb) : tok_group_bytes_hd<64>(kb, vb);
}

int launch_decode_mfma(const DecodeParams& dp_in, int lchunks, int max_kbits, int max_vbits,
                       int waves, bool wave_only, hipStream_t stream) {
  DecodeParams dp = dp_in;
  const int hd = dp.hd;
  // per-token K segments go to the TOK variant (the host never mixes them with KIVI
  // segments or a device table in one launch)
  bool tok = false;
  for (int i = 0; i < dp.nseg; ++i) tok = tok || dp.seg[i].kind == PK_SEG_TOKEN;
  const int maxb = std::max(max_kbits, max_vbits);
  const bool w8 = waves == 8 && maxb <= 4;
  // four waves on the wave-private group path only: a fraction of the full variant's code
  const bool wo = !w8 && !tok && wave_only && maxb <= 4;
  const size_t nw = w8 ? 8 : kWaves;
  size_t staging;
  if (tok) {
    dp.stage_lds = 0;
    staging = nw * 2 * tok_group_bytes(hd, max_kbits, max_vbits);
  } else if (w8 || wo) {
    dp.stage_lds = 0;
    staging = nw * 2 * kivi_group_bytes(hd, max_kbits, max_vbits);
  } else {
    dp.stage_lds = (kivi_stage_bytes(hd, max_kbits, max_vbits) + 15) & ~15;
    staging = std::max(2 * (size_t)dp.stage_lds,
                       (size_t)kWaves * 2 * kivi_group_bytes(hd, max_kbits, max_vbits));
  }
  const size_t merge = sizeof(float) * (nw * 16 * (hd + 4) + 2 * nw * 16);
  const size_t lds = std::max(staging, merge);
  const dim3 grid(lchunks, dp.Hkv * dp.nslab, dp.B);
  if (w8) {
    if (tok) {
      if (hd == 128) return maxb <= 2 ? launch_decode_mfma_tok_w8_128_2(dp, grid, lds, stream)
                                      : launch_decode_mfma_tok_w8_128_4(dp, grid, lds, stream);
      return maxb <= 2 ? launch_decode_mfma_tok_w8_64_2(dp, grid, lds, stream)
                       : launch_decode_mfma_tok_w8_64_4(dp, grid, lds, stream);
    }
    if (hd == 128) return maxb <= 2 ? launch_decode_mfma_w8_128_2(dp, grid, lds, stream)
                                    : launch_decode_mfma_w8_128_4(dp, grid, lds, stream);
    return maxb <= 2 ? launch_decode_mfma_w8_64_2(dp, grid, lds, stream)
                     : launch_decode_mfma_w8_64_4(dp, grid, lds, stream);
  }
  if (wo) {
    if (hd == 128) return maxb <= 2 ? launch_decode_mfma_wo_128_2(dp, grid, lds, stream)
                                    : launch_decode_mfma_wo_128_4(dp, grid, lds, stream);
    return maxb <= 2 ? launch_decode_mfma_wo_64_2(dp, grid, lds, stream)
                     : launch_decode_mfma_wo_64_4(dp, grid, lds, stream);
  }
  if (tok) {
    if (hd == 128) {
      if (maxb <= 2) return launch_decode_mfma_tok_128_2(dp, grid, lds, stream);
      if (maxb <= 4) return launch_decode_mfma_tok_128_4(dp, grid, lds, stream);
      return launch_decode_mfma_tok_128_8(dp, grid, lds, stream);
    }
    if (maxb <= 2) return launch_decode_mfma_tok_64_2(dp, grid, lds, stream);
    if (maxb <= 4) return launch_decode_mfma_tok_64_4(dp, grid, lds, stream);
    return launch_decode_mfma_tok_64_8(dp, grid, lds, stream);
  }
  if (hd == 128) {
    if (maxb <= 2) return launch_decode_mfma_128_2(dp, grid, lds, stream);
    if (maxb <= 4) return launch_decode_mfma_128_4(dp, grid, lds, stream);
    return launch_decode_mfma_128_8(dp, grid, lds, stream);
  }
  if (maxb <= 2) return launch_decode_mfma_64_2(dp, grid, lds, stream);
  if (maxb <= 4) return launch_decode_mfma_64_4(dp, grid, lds, stream);
  return launch_decode_mfma_64_8(dp, grid, lds, stream);
}

}  // namespace pk
