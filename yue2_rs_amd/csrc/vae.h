// vae.h -- the VAE decoder (src/vae.rs) between its checkpoint reader
// (checkpoint.hip) and its device executor (vae.hip).
#pragma once
#include <stdint.h>

#include <vector>

namespace y2 {

enum VaeKind { VAE_CONV = 0, VAE_CONVT = 1, VAE_SNAKE = 2, VAE_ELU = 3, VAE_TANH = 4, VAE_RES_BEGIN = 5,
               VAE_RES_END = 6 };

// One operation of the decoder in network order (network, src/vae.rs:470-546).
// Convolutions: w is the weight-normed kernel in the checkpoint's layout
// ([out, in, k], or [in, out, k] transposed), b the bias (empty: none).
// SnakeBeta: a = exp(alpha), ib = 1 / (exp(beta) + 1e-9) per channel.
struct VaeOpHost {
    int kind = VAE_CONV, cin = 0, cout = 0, kernel = 0, stride = 1, padding = 0, dilation = 1;
    std::vector<float> w, b, a, ib;
};

struct VaeHost {
    std::vector<VaeOpHost> ops;
    int sample_rate = 0, latent_dim = 0, audio_channels = 0, ratio = 0, core_frames = 0, halo_frames = 0;
};

// Vae::open (src/vae.rs:635-669), decoder only: config.json and the
// safetensors file(s) of `dir`, checked as the reference checks them.
// Returns 0 or a negative Yue2Error (message in yue2_hip_last_error).
int vae_read(const char* dir, VaeHost* out);

}  // namespace y2
