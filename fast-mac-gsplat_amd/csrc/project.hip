// project.hip -- pinhole projection of 3D Gaussians to screen-space splats
// and its vector-Jacobian product.  One thread per splat.
//
// Forward (reference project_pinhole_forward,
// variants/v9_project3d_train/csrc/metal/gsplat_v9_project3d_train_kernels.metal:66-174):
//   R = R(q) for q = (r,i,j,k) as given (no normalisation)
//   M = R diag(s), Sigma = M M^T                         (linear scales)
//   W = camera_to_world[:3,:3], t = camera_to_world[:3,3]
//   x_c = W^T (x - t),  Sigma_c = W^T Sigma W
//   front = z_c > near; z_s = front ? z_c : 1; (x_p, y_p) = front ? (x_c, y_c) : 0
//   J = [[fx/z_s, 0, -fx x_p/z_s^2], [0, fy/z_s, -fy y_p/z_s^2]]
//   cov = J Sigma_c J^T + 0.3 I,  det = max(det(cov), 1e-6)
//   conic = (cov11, -cov01, cov00) / det
//   mean2d = (fx x_p/z_s + cx, fy y_p/z_s + cy), opacity' = front ? o : 0,
//   depth = z_c.
// Backward: the chain rule through the same steps written in matrix form
//   dSigma_c = J^T G J, dJ = 2 G J Sigma_c          (G = symmetric dcov)
//   dSigma = W dSigma_c W^T, dW += 2 Sigma W dSigma_c + (x - t) dx_c^T
//   dM = 2 dSigma M, dR = dM diag(s), ds_c = sum_a dM[a][c] R[a][c]
// plus dR/dq; the det clamp blocks the det gradient when it is active
// (reference :338-342).  Camera gradients are summed per workgroup (one
// image per workgroup) into a workspace and reduced by a second launch in a
// fixed order, without atomics.
#include <mutex>

#include "gs_internal.h"

// Camera-gradient partial sums of the allocation-free backward
// (gsplat_hip_project_backward_noalloc): a file-scope device array instead
// of a caller workspace.  Every GPU the library runs on holds its own copy
// until the process ends.  In host code `scratch` names a host-side stand-in,
// not device memory: its device address is looked up once per device
// (project_noalloc_scratch) and only that address is passed to kernels.
static __device__ __align__(256) float scratch[GSPLAT_PROJECT_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace gs {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ void quat_to_rot(float r, float i, float j, float k,
                                            float R[3][3]) {
  R[0][0] = 1.0f - 2.0f * (j * j + k * k);
  R[0][1] = 2.0f * (i * j - r * k);
  R[0][2] = 2.0f * (i * k + r * j);
  R[1][0] = 2.0f * (i * j + r * k);
  R[1][1] = 1.0f - 2.0f * (i * i + k * k);
  R[1][2] = 2.0f * (j * k - r * i);
  R[2][0] = 2.0f * (i * k - r * j);
  R[2][1] = 2.0f * (j * k + r * i);
  R[2][2] = 1.0f - 2.0f * (i * i + j * j);
}

struct Camera {
  float W[3][3];
  float t[3];
  float fx, fy, cx, cy;
};

__device__ __forceinline__ Camera load_camera(const float* c2w,
                                              const float* cam, int b) {
  Camera C;
  const float* m = c2w + 16 * b;
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c) C.W[r][c] = m[4 * r + c];
    C.t[r] = m[4 * r + 3];
  }
  C.fx = cam[4 * b + 0];
  C.fy = cam[4 * b + 1];
  C.cx = cam[4 * b + 2];
  C.cy = cam[4 * b + 3];
  return C;
}

// Forward quantities shared by both kernels.
struct ProjState {
  float R[3][3];      // rotation from the quaternion
  float s[3];         // scales
  float M[3][3];      // R diag(s)
  float Sig[3][3];    // world covariance
  float d[3];         // x - t
  float xc[3];        // camera-space mean
  float Sc[3][3];     // camera-space covariance
  bool front;
  float zs, xp, yp;
  float J[2][3];
  float cov00, cov01, cov11, det_raw, det;
};

__device__ __forceinline__ void project_state(const ProjectParams& P,
                                              const Camera& C,
                                              const float* means3d,
                                              const float* scales,
                                              const float* quats, int gid,
                                              ProjState& S) {
  const float4 q = reinterpret_cast<const float4*>(quats)[gid];
  quat_to_rot(q.x, q.y, q.z, q.w, S.R);
#pragma unroll
  for (int c = 0; c < 3; ++c) S.s[c] = scales[3 * gid + c];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int c = 0; c < 3; ++c) S.M[a][c] = S.R[a][c] * S.s[c];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int b = 0; b < 3; ++b)
      S.Sig[a][b] = S.M[a][0] * S.M[b][0] + S.M[a][1] * S.M[b][1] +
                    S.M[a][2] * S.M[b][2];
#pragma unroll
  for (int a = 0; a < 3; ++a) S.d[a] = means3d[3 * gid + a] - C.t[a];
#pragma unroll
  for (int j = 0; j < 3; ++j)
    S.xc[j] = S.d[0] * C.W[0][j] + S.d[1] * C.W[1][j] + S.d[2] * C.W[2][j];
  // Sc = W^T Sig W
  float SW[3][3];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int q2 = 0; q2 < 3; ++q2)
      SW[a][q2] = S.Sig[a][0] * C.W[0][q2] + S.Sig[a][1] * C.W[1][q2] +
                  S.Sig[a][2] * C.W[2][q2];
#pragma unroll
  for (int p = 0; p < 3; ++p)
#pragma unroll
    for (int q2 = 0; q2 < 3; ++q2)
      S.Sc[p][q2] = C.W[0][p] * SW[0][q2] + C.W[1][p] * SW[1][q2] +
                    C.W[2][p] * SW[2][q2];
  const float z = S.xc[2];
  S.front = z > P.near_plane;
  S.zs = S.front ? fmaxf(z, P.near_plane) : 1.0f;
  S.xp = S.front ? S.xc[0] : 0.0f;
  S.yp = S.front ? S.xc[1] : 0.0f;
  const float iz = 1.0f / S.zs;
  S.J[0][0] = C.fx * iz;
  S.J[0][1] = 0.0f;
  S.J[0][2] = -(C.fx * S.xp) * iz * iz;
  S.J[1][0] = 0.0f;
  S.J[1][1] = C.fy * iz;
  S.J[1][2] = -(C.fy * S.yp) * iz * iz;
  float JS[2][3];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int c = 0; c < 3; ++c)
      JS[r][c] = S.J[r][0] * S.Sc[0][c] + S.J[r][1] * S.Sc[1][c] +
                 S.J[r][2] * S.Sc[2][c];
  S.cov00 = JS[0][0] * S.J[0][0] + JS[0][1] * S.J[0][1] +
            JS[0][2] * S.J[0][2] + 0.3f;
  S.cov01 = JS[0][0] * S.J[1][0] + JS[0][1] * S.J[1][1] +
            JS[0][2] * S.J[1][2];
  S.cov11 = JS[1][0] * S.J[1][0] + JS[1][1] * S.J[1][1] +
            JS[1][2] * S.J[1][2] + 0.3f;
  S.det_raw = S.cov00 * S.cov11 - S.cov01 * S.cov01;
  S.det = fmaxf(S.det_raw, 1e-6f);
}

__global__ __launch_bounds__(kThreads) void project_fwd_kernel(
    ProjectParams P, const float* __restrict__ means3d,
    const float* __restrict__ scales, const float* __restrict__ quats,
    const float* __restrict__ opacities, const float* __restrict__ c2w,
    const float* __restrict__ cam, float* __restrict__ out_means2d,
    float* __restrict__ out_conics, float* __restrict__ out_opac,
    float* __restrict__ out_depths) {
  const int gid = blockIdx.x * kThreads + threadIdx.x;
  if (gid >= P.num_splats) return;
  const int b = gid / P.gpb;
  const Camera C = load_camera(c2w, cam, b);
  ProjState S;
  project_state(P, C, means3d, scales, quats, gid, S);
  out_means2d[2 * gid + 0] = (C.fx * S.xp) / S.zs + C.cx;
  out_means2d[2 * gid + 1] = (C.fy * S.yp) / S.zs + C.cy;
  out_conics[3 * gid + 0] = S.cov11 / S.det;
  out_conics[3 * gid + 1] = -S.cov01 / S.det;
  out_conics[3 * gid + 2] = S.cov00 / S.det;
  out_opac[gid] = S.front ? opacities[gid] : 0.0f;
  out_depths[gid] = S.xc[2];
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__global__ __launch_bounds__(kThreads) void project_bwd_kernel(
    ProjectParams P, const float* __restrict__ g_means2d,
    const float* __restrict__ g_conics, const float* __restrict__ g_opac_out,
    const float* __restrict__ g_depths, const float* __restrict__ means3d,
    const float* __restrict__ scales, const float* __restrict__ quats,
    const float* __restrict__ opacities, const float* __restrict__ c2w,
    const float* __restrict__ cam, float* __restrict__ out_g_means3d,
    float* __restrict__ out_g_scales, float* __restrict__ out_g_quats,
    float* __restrict__ out_g_opac, float* __restrict__ cam_partials) {
  // Workgroup (x, b) handles splats x*256 .. x*256+255 of image b, so its
  // camera-gradient partial sums belong to one camera.
  const int b = blockIdx.y;
  const int local = blockIdx.x * kThreads + threadIdx.x;
  const bool active = local < P.gpb;
  const int g = b * P.gpb + (active ? local : (P.gpb - 1));
  const Camera C = load_camera(c2w, cam, b);
  ProjState S;
  project_state(P, C, means3d, scales, quats, g, S);

  // ---- conic -> cov2d
  const float gq0 = g_conics[3 * g + 0];
  const float gq1 = g_conics[3 * g + 1];
  const float gq2 = g_conics[3 * g + 2];
  const float idet = 1.0f / S.det;
  float g00 = gq2 * idet;
  float g11 = gq0 * idet;
  float g01 = -gq1 * idet;  // d/d(cov01) treating cov01 as one variable
  if (S.det_raw > 1e-6f) {
    const float gdet =
        -(gq0 * S.cov11 - gq1 * S.cov01 + gq2 * S.cov00) * idet * idet;
    g00 += gdet * S.cov11;
    g11 += gdet * S.cov00;
    g01 += gdet * (-2.0f * S.cov01);
  }
  // Symmetric matrix gradient of cov (off-diagonals split evenly).
  const float G[2][2] = {{g00, 0.5f * g01}, {0.5f * g01, g11}};

  // ---- cov = J Sc J^T:  dSc = J^T G J,  dJ = 2 G J Sc
  float GJ[2][3];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int c = 0; c < 3; ++c)
      GJ[r][c] = G[r][0] * S.J[0][c] + G[r][1] * S.J[1][c];
  float dSc[3][3];
#pragma unroll
  for (int p = 0; p < 3; ++p)
#pragma unroll
    for (int q2 = 0; q2 < 3; ++q2)
      dSc[p][q2] = S.J[0][p] * GJ[0][q2] + S.J[1][p] * GJ[1][q2];
  float dJ[2][3];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int c = 0; c < 3; ++c)
      dJ[r][c] = 2.0f * (GJ[r][0] * S.Sc[0][c] + GJ[r][1] * S.Sc[1][c] +
                         GJ[r][2] * S.Sc[2][c]);

  // ---- J, mean2d -> camera-space mean and intrinsics
  const float gmx = g_means2d[2 * g + 0];
  const float gmy = g_means2d[2 * g + 1];
  float gxc[3] = {0.0f, 0.0f, g_depths != nullptr ? g_depths[g] : 0.0f};
  float g_fx = 0.0f, g_fy = 0.0f;
  const float g_cx = gmx, g_cy = gmy;
  if (S.front) {
    const float x = S.xc[0], y = S.xc[1], z = S.xc[2];
    const float iz = 1.0f / z, iz2 = iz * iz, iz3 = iz2 * iz;
    g_fx += gmx * x * iz;
    gxc[0] += gmx * C.fx * iz;
    gxc[2] -= gmx * C.fx * x * iz2;
    g_fy += gmy * y * iz;
    gxc[1] += gmy * C.fy * iz;
    gxc[2] -= gmy * C.fy * y * iz2;
    // J00 = fx/z, J02 = -fx x/z^2, J11 = fy/z, J12 = -fy y/z^2
    g_fx += dJ[0][0] * iz - dJ[0][2] * x * iz2;
    g_fy += dJ[1][1] * iz - dJ[1][2] * y * iz2;
    gxc[0] -= dJ[0][2] * C.fx * iz2;
    gxc[1] -= dJ[1][2] * C.fy * iz2;
    gxc[2] += -dJ[0][0] * C.fx * iz2 + 2.0f * dJ[0][2] * C.fx * x * iz3 -
              dJ[1][1] * C.fy * iz2 + 2.0f * dJ[1][2] * C.fy * y * iz3;
  } else {
    // z_s = 1 and x_p = y_p = 0: J00 = fx, J11 = fy, J02 = J12 = 0.
    g_fx += dJ[0][0];
    g_fy += dJ[1][1];
  }

  // ---- x_c = W^T d, Sc = W^T Sig W
  float gW[3][3];
  float gmean[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    gmean[a] = C.W[a][0] * gxc[0] + C.W[a][1] * gxc[1] + C.W[a][2] * gxc[2];
#pragma unroll
    for (int j = 0; j < 3; ++j) gW[a][j] = S.d[a] * gxc[j];
  }
  // dSig = W dSc W^T ; dW += 2 Sig W dSc
  float WdS[3][3];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int q2 = 0; q2 < 3; ++q2)
      WdS[a][q2] = C.W[a][0] * dSc[0][q2] + C.W[a][1] * dSc[1][q2] +
                   C.W[a][2] * dSc[2][q2];
  float dSig[3][3];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int bb = 0; bb < 3; ++bb)
      dSig[a][bb] = WdS[a][0] * C.W[bb][0] + WdS[a][1] * C.W[bb][1] +
                    WdS[a][2] * C.W[bb][2];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int q2 = 0; q2 < 3; ++q2)
      gW[a][q2] += 2.0f * (S.Sig[a][0] * WdS[0][q2] + S.Sig[a][1] * WdS[1][q2] +
                           S.Sig[a][2] * WdS[2][q2]);

  // ---- Sig = M M^T, M = R diag(s)
  float dM[3][3];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int c = 0; c < 3; ++c)
      dM[a][c] = 2.0f * (dSig[a][0] * S.M[0][c] + dSig[a][1] * S.M[1][c] +
                         dSig[a][2] * S.M[2][c]);
  float gs[3];
  float dR[3][3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    gs[c] = dM[0][c] * S.R[0][c] + dM[1][c] * S.R[1][c] + dM[2][c] * S.R[2][c];
#pragma unroll
    for (int a = 0; a < 3; ++a) dR[a][c] = dM[a][c] * S.s[c];
  }
  const float4 q = reinterpret_cast<const float4*>(quats)[g];
  const float qr = q.x, qi = q.y, qj = q.z, qk = q.w;
  // dR/dq for R(q) as in quat_to_rot.
  const float gqr = 2.0f * (-qk * dR[0][1] + qj * dR[0][2] + qk * dR[1][0] -
                            qi * dR[1][2] - qj * dR[2][0] + qi * dR[2][1]);
  const float gqi = 2.0f * (qj * dR[0][1] + qk * dR[0][2] + qj * dR[1][0] -
                            qr * dR[1][2] + qk * dR[2][0] + qr * dR[2][1]) -
                    4.0f * qi * (dR[1][1] + dR[2][2]);
  const float gqj = 2.0f * (qi * dR[0][1] + qr * dR[0][2] + qi * dR[1][0] +
                            qk * dR[1][2] - qr * dR[2][0] + qk * dR[2][1]) -
                    4.0f * qj * (dR[0][0] + dR[2][2]);
  const float gqk = 2.0f * (-qr * dR[0][1] + qi * dR[0][2] + qr * dR[1][0] +
                            qj * dR[1][2] + qi * dR[2][0] + qj * dR[2][1]) -
                    4.0f * qk * (dR[0][0] + dR[1][1]);

  if (active) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      out_g_means3d[3 * g + a] = gmean[a];
      out_g_scales[3 * g + a] = gs[a];
    }
    reinterpret_cast<float4*>(out_g_quats)[g] = make_float4(gqr, gqi, gqj, gqk);
    out_g_opac[g] = S.front ? g_opac_out[g] : 0.0f;
  }

  // ---- camera gradients: 9 rotation + 3 translation + 4 intrinsics
  float cv[16];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int j = 0; j < 3; ++j) cv[3 * a + j] = active ? gW[a][j] : 0.0f;
#pragma unroll
  for (int a = 0; a < 3; ++a) cv[9 + a] = active ? -gmean[a] : 0.0f;
  cv[12] = active ? g_fx : 0.0f;
  cv[13] = active ? g_fy : 0.0f;
  cv[14] = active ? g_cx : 0.0f;
  cv[15] = active ? g_cy : 0.0f;
  // Workgroup sum of the 16 values -> cam_partials[(b * nbx + x) * 16 + v].
  __shared__ float part[kThreads / 64][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const float sv = wave_sum(cv[v]);
    if (lane == 0) part[wave][v] = sv;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) sum += part[w][threadIdx.x];
    cam_partials[((int64_t)b * gridDim.x + blockIdx.x) * 16 + threadIdx.x] = sum;
  }
}

// One workgroup per image: sums the nbx workgroup partials of each of the 16
// camera-gradient values (fixed order, no atomics) and writes
// g_camera_to_world [B,4,4] (rotation 3x3, translation column, zero last row)
// and g_camera_params [B,4].  64 slots of 16 threads read rows slot, slot +
// 64, ... with four independent sums (so four loads are in flight per
// thread), then a fixed tree over the slots.
constexpr int kReduceThreads = 1024;
constexpr int kReduceSlots = kReduceThreads / 16;
__global__ __launch_bounds__(kReduceThreads) void project_cam_reduce_kernel(
    const float* __restrict__ cam_partials, int nbx, float* __restrict__ g_c2w,
    float* __restrict__ g_cam) {
  __shared__ float red[kReduceThreads];
  const int b = blockIdx.x;
  const int v = threadIdx.x & 15, slot = threadIdx.x >> 4;
  const float* rows = cam_partials + (int64_t)b * nbx * 16 + v;
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
  int x = slot;
  for (; x + 3 * kReduceSlots < nbx; x += 4 * kReduceSlots) {
    s0 += rows[(int64_t)x * 16];
    s1 += rows[(int64_t)(x + kReduceSlots) * 16];
    s2 += rows[(int64_t)(x + 2 * kReduceSlots) * 16];
    s3 += rows[(int64_t)(x + 3 * kReduceSlots) * 16];
  }
  for (; x < nbx; x += kReduceSlots) s0 += rows[(int64_t)x * 16];
  red[threadIdx.x] = (s0 + s1) + (s2 + s3);
  __syncthreads();
#pragma unroll
  for (int w = kReduceSlots / 2; w >= 1; w >>= 1) {
    if (slot < w) red[threadIdx.x] += red[threadIdx.x + 16 * w];
    __syncthreads();
  }
  if (threadIdx.x < 16) {
    const float total = red[v];
    float* gc2w = g_c2w + 16 * b;
    if (v < 9) gc2w[4 * (v / 3) + (v % 3)] = total;        // rotation
    else if (v < 12) gc2w[4 * (v - 9) + 3] = total;         // translation
    else g_cam[4 * b + (v - 12)] = total;                   // fx, fy, cx, cy
    if (v < 4) gc2w[12 + v] = 0.0f;                         // last row
  }
}

}  // namespace

int launch_project_forward(const ProjectParams& P, const float* means3d,
                           const float* scales, const float* quats,
                           const float* opacities, const float* c2w,
                           const float* cam, float* out_means2d,
                           float* out_conics, float* out_opac,
                           float* out_depths, hipStream_t stream) {
  if (P.num_splats == 0) return GSPLAT_OK;
  const unsigned grid = (unsigned)((P.num_splats + kThreads - 1) / kThreads);
  launch_traced("project_fwd_kernel", project_fwd_kernel, dim3(grid),
                dim3(kThreads), 0, stream, P, means3d, scales, quats, opacities,
                c2w, cam, out_means2d, out_conics, out_opac, out_depths);
  return check_launch("project_fwd_kernel");
}

namespace {
constexpr int kMaxDevices = 256;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device
}  // namespace

int project_noalloc_scratch(hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    set_error("project_backward_noalloc: cannot resolve the stream's device (%s)",
              e != hipSuccess ? hipGetErrorString(e) : "device index out of range");
    return GSPLAT_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    // hipGetSymbolAddress resolves the symbol on the current device: make the
    // stream's device current for the lookup and restore the caller's after.
    int cur = 0;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      set_error("project_backward_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                e != hipSuccess ? hipGetErrorString(e) : "null address");
      return GSPLAT_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GSPLAT_OK;
}

size_t project_backward_workspace_bytes(const ProjectParams& P) {
  const int64_t nbx = (P.gpb + kThreads - 1) / kThreads;
  return align_up((size_t)(P.batch * nbx * 16) * sizeof(float), 256);
}

int launch_project_backward(const ProjectParams& P, const float* g_means2d,
                            const float* g_conics, const float* g_opac_out,
                            const float* g_depths, const float* means3d,
                            const float* scales, const float* quats,
                            const float* opacities, const float* c2w,
                            const float* cam, float* g_means3d,
                            float* g_scales, float* g_quats, float* g_opac,
                            float* g_c2w, float* g_cam, void* workspace,
                            hipStream_t stream) {
  if (P.num_splats == 0) {
    int rc = launch_fill_f32(g_c2w, 0.0f, 16 * (int64_t)P.batch, stream);
    if (!rc) rc = launch_fill_f32(g_cam, 0.0f, 4 * (int64_t)P.batch, stream);
    return rc;
  }
  const int nbx = (P.gpb + kThreads - 1) / kThreads;
  float* partials = static_cast<float*>(workspace);
  launch_traced("project_bwd_kernel", project_bwd_kernel,
                dim3((unsigned)nbx, (unsigned)P.batch), dim3(kThreads), 0,
                stream, P, g_means2d, g_conics, g_opac_out, g_depths, means3d,
                scales, quats, opacities, c2w, cam, g_means3d, g_scales,
                g_quats, g_opac, partials);
  int rc = check_launch("project_bwd_kernel");
  if (rc) return rc;
  launch_traced("project_cam_reduce_kernel", project_cam_reduce_kernel,
                dim3((unsigned)P.batch), dim3(kReduceThreads), 0, stream,
                partials, nbx, g_c2w, g_cam);
  return check_launch("project_cam_reduce_kernel");
}

}  // namespace gs
