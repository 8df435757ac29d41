"""Build libadhip.so in-tree with hipcc for gfx950 (``python -m ad_amd.build``)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
SRCS = [os.path.join(ROOT, "csrc", f) for f in ("adhip.cpp", "adhip_colreduce.cpp")]
OUT = os.path.join(ROOT, "device", "hip", "libadhip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = ["-O2", "-fPIC", "-shared", "-std=c++17", "--offload-arch=gfx950",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def build_library(verbose=False) -> str:
    tmp = OUT + f".tmp{os.getpid()}"
    cmd = [HIPCC, *FLAGS, *SRCS, "-o", tmp, "-lhiprtc"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print("built", OUT)
    return OUT


def check_templates() -> None:
    """Compile one instance of every device template for gfx950 through
    hipRTC (the path kernels take at run time)."""
    sys.path.insert(0, os.path.dirname(ROOT))
    from ad_amd.device.hip.runtime import HEADER_PATH, compile_source
    with open(HEADER_PATH) as fh:
        header = fh.read()
    probe = r'''
struct LA { static constexpr int kMode = 0; static constexpr bool kVec = true; float* p0;
  __device__ float at(unsigned x, unsigned y) const { return p0[x * 64u + y]; }
  __device__ float4 at4(unsigned x, unsigned y) const { return *reinterpret_cast<const float4*>(p0 + x * 64u + y); } };
struct LB { static constexpr int kMode = 1; static constexpr bool kVec = false; float* p0;
  __device__ float at(unsigned x, unsigned y) const { return p0[y * 64u + x]; }
  __device__ float4 at4(unsigned x, unsigned y) const { return *reinterpret_cast<const float4*>(p0 + y * 64u + x); } };
struct EPI { float* p0; static constexpr bool kVec4 = false; static constexpr int kLoads = 1;
  __device__ void load(unsigned x, unsigned y, float* l) const { l[0] = p0[x * 64u + y]; }
  __device__ void operator()(float v, unsigned x, unsigned y, int c, const float* l) const { p0[(c * 64u + x) * 64u + y] = v + l[0]; } };
struct EP4 { float* p0; static constexpr bool kVec4 = true; static constexpr int kLoads = 1;
  __device__ void load4(unsigned x, unsigned y, float4* l) const { l[0] = *reinterpret_cast<const float4*>(p0 + x * 64u + y); }
  __device__ void vec(float4 v, unsigned x, unsigned y, int c, const float4* l) const {
    *reinterpret_cast<float4*>(p0 + (c * 64u + x) * 64u + y) = make_float4(v.x + l[0].x, v.y + l[0].y, v.z + l[0].z, v.w + l[0].w); } };
struct LD { static constexpr bool kVec = true; static constexpr bool kVecX = false; float* p0;
  __device__ float at(unsigned x, unsigned y) const { return p0[x * 64u + y]; }
  __device__ float4 at4(unsigned x, unsigned y) const { return *reinterpret_cast<const float4*>(p0 + x * 64u + y); }
  __device__ bool inc(unsigned) const { return true; } };
struct LDX { static constexpr bool kVec = false; static constexpr bool kVecX = true; float* p0;
  __device__ float at(unsigned x, unsigned y) const { return p0[y * 64u + x]; }
  __device__ float4 at4(unsigned x, unsigned y) const { return *reinterpret_cast<const float4*>(p0 + y * 64u + x); }
  __device__ bool inc(unsigned) const { return true; } };
struct EPR { float* p0; __device__ void operator()(float v, unsigned x, int c) const { p0[c * 64u + x] = v; } };
extern "C" __global__ void __launch_bounds__(256) probe_dp(float* a) { adhip::dp_mfma<128, 128, 1, 16>(LA{a}, LB{a}, EPI{a}, 64, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_dp_narrow(float* a) { adhip::dp_mfma<128, 64, 4, 32>(LA{a}, LB{a}, EPI{a}, 64, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_dp_small(float* a) { adhip::dp_mfma<64, 64, 2, 16>(LA{a}, LB{a}, EPI{a}, 64, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_dp_vec(float* a) { adhip::dp_mfma<128, 64, 1, 16>(LA{a}, LB{a}, EP4{a}, 64, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_dp_vec_small(float* a) { adhip::dp_mfma<64, 64, 4, 64>(LA{a}, LB{a}, EP4{a}, 64, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_quad(float* a) { adhip::dp_quad<1, 128>(LA{a}, LB{a}, EPI{a}, 64, 64, 256); }
extern "C" __global__ void __launch_bounds__(256) probe_quad_vec(float* a) { adhip::dp_quad<8, 128>(LA{a}, LB{a}, EP4{a}, 64, 64, 4096); }
extern "C" __global__ void __launch_bounds__(256) probe_quad_short(float* a) { adhip::dp_quad<1, 64>(LA{a}, LB{a}, EP4{a}, 64, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_pack(float* a) { adhip::pack_bf16<0>(LA{a}, reinterpret_cast<__bf16*>(a), 64, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_pack_t(float* a) { adhip::pack_bf16<1>(LB{a}, reinterpret_cast<__bf16*>(a), 64, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_bf16(float* a) { adhip::dp_bf16<128, 128, 1, 64>(reinterpret_cast<const __bf16*>(a), reinterpret_cast<const __bf16*>(a), 64, EP4{a}, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_direct(float* a) { adhip::dp_direct(LA{a}, LB{a}, EPI{a}, 64, 64, 2); }
extern "C" __global__ void __launch_bounds__(256) probe_skinny(float* a) { adhip::dp_skinny<8>(LA{a}, LB{a}, EPI{a}, 2, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_bf16_w(float* a) { adhip::dp_bf16<256, 128, 2, 32>(reinterpret_cast<const __bf16*>(a), reinterpret_cast<const __bf16*>(a), 64, EP4{a}, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_bf16_s(float* a) { adhip::dp_bf16<64, 64, 2, 32>(reinterpret_cast<const __bf16*>(a), reinterpret_cast<const __bf16*>(a), 64, EPI{a}, 64, 64); }
extern "C" __global__ void __launch_bounds__(256) probe_rr(float* a) { adhip::reduce_rows<0>(LD{a}, EPR{a}, 64u, 64u, false); }
extern "C" __global__ void __launch_bounds__(256) probe_rc(float* a) { adhip::reduce_cols<1, 1>(LD{a}, EPR{a}, 64u, 64u, true); }
extern "C" __global__ void __launch_bounds__(256) probe_rcs(float* a) { adhip::reduce_cols<0, 8>(LD{a}, EPR{a}, 64u, 64u, false); }
extern "C" __global__ void __launch_bounds__(256) probe_rcv(float* a) { adhip::reduce_cols<0, 8>(LDX{a}, EPR{a}, 64u, 64u, false); }
'''
    compile_source(header + probe)


if __name__ == "__main__":
    build_library(verbose=True)
    check_templates()
    print("templates ok")
