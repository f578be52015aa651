//! The HIP backend (feature `hip`): device buffers and the kernels of kernels/hip (this repository's det_amd/csrc)
//! through det-sys, for AMD Instinct MI355X.  It follows the CUDA backend's shape (reference crates/det/src/cuda.rs)
//! with three differences:
//!   * `linear` uploads the fused det rows once and lets det_linear_repack write this backend's private layout on
//!     the device (K-tiled, coalesced decode tiles plus the prefill planes) instead of splitting rows on the host;
//!   * no caller scratch: the HIP GEMM needs none (det_gemm_set_scratch is accepted and unused);
//!   * sampling with temperature / top-k / top-p is out of this backend's scope: the logits are read back and the
//!     reference CPU backend samples them (greedy decoding uses det_argmax on the device).
//! UNVERIFIED: no Rust toolchain was available where this was written; the C entry points it calls are exercised
//! through ctypes by the repository's tests.

use crate::backend::*;
use crate::gguf::{Gguf, TensorInfo};
use det_sys as ffi;
use std::cell::RefCell;
use std::ffi::{c_int, c_void, CStr};
use std::ptr::null_mut;
use std::sync::Arc;

const ST: ffi::Stream = null_mut();

pub struct Hip {
    attn_scratch: RefCell<Option<Buf<u8>>>,
    gdn_scratch: RefCell<Option<Buf<u8>>>,
    pick: Buf<c_int>,
}

/// The planes det_linear_repack writes (layout private to this backend, documented in det_hip.h).
pub struct HipLinear {
    wq: Buf<u8>,
    c: Buf<f32>,
    m: Buf<u16>,
    widths: Vec<usize>,
    n: usize,
    k: usize,
    bits: u32,
}

unsafe fn release(p: *mut u8) {
    ffi::det_free(p as *mut c_void);
}

fn device_buf<T: Copy>(len: usize) -> Buf<T> {
    let bytes = (len * std::mem::size_of::<T>()).max(16);
    let p = unsafe { ffi::det_malloc(bytes) };
    assert!(!p.is_null(), "det_malloc({bytes}) failed");
    unsafe { Buf::from_device(p as *mut T, len, release) }
}

impl crate::hooks::Reader for Hip {
    unsafe fn read_bytes(&self, src: *const u8, bytes: usize, out: &mut [u8]) {
        unsafe {
            ffi::det_memcpy(out.as_mut_ptr() as *mut c_void, src as *const c_void, bytes, ST);
            ffi::det_sync();
        }
    }
}

impl Hip {
    pub fn new() -> Self {
        assert_eq!(unsafe { ffi::det_init() }, 0, "HIP runtime failed to initialize");
        Hip { attn_scratch: RefCell::new(None), gdn_scratch: RefCell::new(None), pick: device_buf(1) }
    }

    pub fn allocated_bytes() -> usize {
        unsafe { ffi::det_allocated_bytes() }
    }

    fn scratch(slot: &RefCell<Option<Buf<u8>>>, bytes: usize) -> *mut c_void {
        let mut s = slot.borrow_mut();
        if s.as_ref().is_none_or(|b| b.len() < bytes) {
            *s = Some(device_buf(bytes.max(256)));
        }
        s.as_ref().unwrap().as_mut_ptr() as *mut c_void
    }

    fn qlinear(lin: &HipLinear) -> ffi::QLinear {
        ffi::hip::qlinear(lin.wq.as_ptr(), lin.c.as_ptr(), lin.m.as_ptr(), lin.n, lin.k, lin.bits)
    }
}

impl Default for Hip {
    fn default() -> Self {
        Self::new()
    }
}

impl Backend for Hip {
    type Linear = HipLinear;

    fn name(&self) -> String {
        unsafe { CStr::from_ptr(ffi::det_device_name()).to_string_lossy().into_owned() }
    }
    fn alloc<T: Copy>(&self, len: usize) -> Buf<T> {
        device_buf(len)
    }
    fn write<T: Copy>(&self, b: &Buf<T>, offset: usize, data: &[T]) {
        assert!(offset + data.len() <= b.len());
        unsafe {
            ffi::det_memcpy(b.ptr_at(offset) as *mut c_void, data.as_ptr() as *const c_void, std::mem::size_of_val(data), ST)
        }
    }
    fn read<T: Copy>(&self, b: &Buf<T>, offset: usize, out: &mut [T]) {
        assert!(offset + out.len() <= b.len());
        unsafe {
            ffi::det_memcpy(out.as_mut_ptr() as *mut c_void, b.ptr_at(offset) as *const c_void, std::mem::size_of_val(out), ST);
            ffi::det_sync();
        }
    }
    fn zero<T: Copy>(&self, b: &Buf<T>) {
        unsafe { ffi::det_memset(b.as_mut_ptr() as *mut c_void, 0, b.bytes(), ST) }
    }
    fn sync(&self) {
        unsafe { ffi::det_sync() }
    }

    /// The fused parts' det rows (model.rs:180-197) go to the device as they are; det_linear_repack writes the
    /// decode tiles and prefill planes there, and the rows are released.
    fn linear(&self, g: &Arc<Gguf>, parts: &[&TensorInfo]) -> HipLinear {
        let cpu = crate::cpu::linear_parts(g, parts);
        let (bits, k) = (cpu.bits, cpu.k);
        let n = cpu.widths.iter().sum::<usize>();
        let rb = crate::spec::det_row_bytes(bits, k);
        let mut rows = vec![0u8; n * rb];
        for (r, dst) in rows.chunks_mut(rb).enumerate() {
            dst.copy_from_slice(&cpu.row(r)[..rb]);
        }
        let dev_rows: Buf<u8> = self.upload(&rows);
        drop(rows);
        let (mut wb, mut cb, mut mb) = (0usize, 0usize, 0usize);
        unsafe { ffi::hip::det_linear_sizes(n as c_int, k as c_int, bits as c_int, &mut wb, &mut cb, &mut mb) };
        let (wq, c, m): (Buf<u8>, Buf<f32>, Buf<u16>) = (device_buf(wb), device_buf(cb / 4), device_buf(mb / 2));
        unsafe {
            ffi::hip::det_linear_repack(dev_rows.as_ptr(), n as c_int, k as c_int, bits as c_int, wq.as_mut_ptr(),
                                        c.as_mut_ptr(), m.as_mut_ptr(), ST);
        }
        drop(dev_rows);                        // det_free waits for the repack
        HipLinear { wq, c, m, widths: cpu.widths.clone(), n, k, bits }
    }
    fn linear_widths(lin: &HipLinear) -> &[usize] {
        &lin.widths
    }

    fn rmsnorm_quant(&self, x: &Buf<f32>, w: &Buf<f32>, eps: f32, m: usize, n: usize, xq: &Buf<i8>, sx: &Buf<f32>,
                     mx: &Buf<u16>) {
        unsafe {
            ffi::det_rmsnorm_quant(x.as_ptr(), w.as_ptr(), eps, m as c_int, n as c_int, null_mut(), xq.as_mut_ptr(),
                                   sx.as_mut_ptr(), mx.as_mut_ptr(), ST)
        }
    }

    fn quant(&self, x: &Buf<f32>, m: usize, n: usize, xq: &Buf<i8>, sx: &Buf<f32>, mx: &Buf<u16>) {
        unsafe { ffi::det_quant(x.as_ptr(), m as c_int, n as c_int, xq.as_mut_ptr(), sx.as_mut_ptr(), mx.as_mut_ptr(), ST) }
    }

    fn gemm(&self, lin: &HipLinear, xq: &Buf<i8>, sx: &Buf<f32>, mx: &Buf<u16>, m: usize, out: GemmOut) {
        let q = Self::qlinear(lin);
        let (xp, sp, mp, mm) = (xq.as_ptr(), sx.as_ptr(), mx.as_ptr(), m as c_int);
        unsafe {
            match out {
                GemmOut::Write(y) => {
                    ffi::det_gemm_ex(&q, xp, sp, mp, mm, y.as_mut_ptr(), 0, 0, std::ptr::null(), std::ptr::null(), ST)
                }
                GemmOut::Accumulate(y) => {
                    ffi::det_gemm_ex(&q, xp, sp, mp, mm, y.as_mut_ptr(), 1, 0, std::ptr::null(), std::ptr::null(), ST)
                }
                GemmOut::Parts(dsts) => {
                    assert_eq!(dsts.len(), lin.widths.len());
                    let offs: Vec<c_int> = lin
                        .widths
                        .iter()
                        .scan(0usize, |acc, w| {
                            let o = *acc;
                            *acc += w;
                            Some(o as c_int)
                        })
                        .collect();
                    let ptrs: Vec<*mut f32> = dsts.iter().map(|d| d.as_mut_ptr()).collect();
                    ffi::det_gemm_ex(&q, xp, sp, mp, mm, null_mut(), 0, dsts.len() as c_int, offs.as_ptr(), ptrs.as_ptr(), ST)
                }
            }
        }
    }

    fn silu_mul_quant(&self, g: &Buf<f32>, u: &Buf<f32>, m: usize, n: usize, hq: &Buf<i8>, sh: &Buf<f32>,
                      mh: &Buf<u16>) {
        unsafe {
            ffi::det_silu_mul_quant(g.as_ptr(), u.as_ptr(), m as c_int, n as c_int, null_mut(), hq.as_mut_ptr(),
                                    sh.as_mut_ptr(), mh.as_mut_ptr(), ST)
        }
    }

    fn attention(&self, l: &AttnLayer, kv: &KvCache, s: &Shape, qg: &Buf<f32>, k: &Buf<f32>, v: &Buf<f32>, o: &Buf<f32>) {
        let layer = ffi::AttnLayer {
            q_norm: l.q_norm.as_ptr(),
            k_norm: l.k_norm.as_ptr(),
            v_scale: l.v_scale.as_ptr(),
            v_inv_scale: l.v_inv_scale.as_ptr(),
        };
        let cache = ffi::KvCache {
            kq: kv.kq.as_mut_ptr(),
            sk: kv.sk.as_mut_ptr(),
            vq: kv.vq.as_mut_ptr(),
            capacity: kv.capacity as c_int,
            vlo: null_mut(),
            vhi: null_mut(),
        };
        let bytes = unsafe { ffi::det_attn_scratch_bytes(s.m as c_int, s.n_h as c_int, s.hd as c_int) };
        let scratch = Self::scratch(&self.attn_scratch, bytes);
        unsafe {
            ffi::det_attention(&layer, &cache, qg.as_ptr(), k.as_ptr(), v.as_ptr(), l.rope_cos.as_ptr(),
                               l.rope_sin.as_ptr(), s.rot as c_int, s.eps, s.m as c_int, s.pos0 as c_int,
                               s.n_h as c_int, s.n_kv as c_int, s.hd as c_int, o.as_mut_ptr(), scratch, ST)
        }
    }

    fn gdn(&self, l: &GdnLayer, st: &GdnState, s: &GdnShape, qkv: &Buf<f32>, z: &Buf<f32>, a: &Buf<f32>, b: &Buf<f32>,
           on: &Buf<f32>, ex: GdnExport) {
        assert!(ex.gin.is_none() && ex.gout.is_none(), "the hip backend does not export GDN gates (det calibrate)");
        let layer = ffi::GdnLayer {
            conv: l.conv.as_ptr(),
            a: l.a.as_ptr(),
            dt_bias: l.dt_bias.as_ptr(),
            norm: l.norm.as_ptr(),
        };
        let mut state = ffi::GdnState { conv_state: st.conv_state.as_mut_ptr(), s: st.s.as_mut_ptr() };
        let bytes = unsafe {
            ffi::det_gdn_scratch_bytes(s.m as c_int, s.n_k as c_int, s.n_v as c_int, s.dk as c_int, s.dv as c_int)
        };
        let scratch = Self::scratch(&self.gdn_scratch, bytes);
        unsafe {
            ffi::det_gdn(&layer, &mut state, qkv.as_ptr(), z.as_ptr(), a.as_ptr(), b.as_ptr(), s.eps, s.m as c_int,
                         s.n_k as c_int, s.n_v as c_int, s.dk as c_int, s.dv as c_int, on.as_mut_ptr(), scratch, ST)
        }
    }

    fn argmax(&self, logits: &Buf<f32>, v: usize) -> i32 {
        unsafe { ffi::det_argmax(logits.as_ptr(), 1, v as c_int, self.pick.as_mut_ptr(), ST) };
        self.download(&self.pick)[0]
    }

    /// Temperature / top-k / top-p sampling is outside this backend: the reference CPU backend samples the logits.
    fn sample(&self, logits: &Buf<f32>, v: usize, inv_temp: f32, top_k: usize, top_p: f32, z: u64) -> i32 {
        let host = Buf::host_from(&self.download(logits)[..v]);
        crate::cpu::Cpu.sample(&host, v, inv_temp, top_k, top_p, z)
    }
}

/// The elementwise primitive test hook (`det_test_prim`): `op` as in det_hip.h.
pub fn test_prim(op: i32, x: &[f32], m: usize, n: usize) -> Vec<f32> {
    let b = Hip::new();
    let xb: Buf<f32> = b.upload(x);
    let out: Buf<f32> = device_buf(x.len().max(m));
    unsafe { ffi::det_test_prim(op, xb.as_ptr(), m as c_int, n as c_int, out.as_mut_ptr(), ST) };
    b.download(&out)
}
