//! `Hip`: det's `Backend` (reference crates/det/src/backend.rs:203-302) on AMD Instinct MI355X, over the C API of
//! include/det_hip.h (kernels compiled from det_amd/csrc by det-sys's `hip` feature).
//!
//! Design, and where it departs from the other GPU backends:
//!   * Weights: `linear` sends the fused det rows (model.rs:180-197) to the device once and the library's
//!     det_linear_repack lays them out in its private K-tiled form; the staging rows are released afterwards.  No
//!     host-side row split happens.
//!   * Workspace: one device arena serves every op that needs temporary memory (attention, Gated DeltaNet and the
//!     one-int result of argmax).  det runs every op on one in-order stream, so consecutive ops can share it; it
//!     grows to the largest request and is replaced, never shrunk.  The GEMM takes no caller scratch.
//!   * Sampling with temperature / top-k / top-p is outside this backend: the logits are read back and the host
//!     backend samples them.  Greedy decoding stays on the device (det_argmax).
//! UNVERIFIED: no Rust toolchain was available where this was written; every C entry point it calls is exercised
//! through ctypes by the repository's tests.

use crate::backend::*;
use crate::gguf::{Gguf, TensorInfo};
use det_sys as sys;
use std::cell::Cell;
use std::ffi::{c_int, c_void, CStr};
use std::mem::size_of;
use std::ptr::{null, null_mut};
use std::sync::Arc;

/// det's stream: the null stream (det_hip_stream returns it).
const STREAM: sys::Stream = null_mut();

/// Bytes at the start of the workspace kept for small results read back by the host (argmax's index).
const RESULT_BYTES: usize = 256;

fn ci(v: usize) -> c_int {
    c_int::try_from(v).expect("dimension exceeds the C API's int range")
}

unsafe fn free_device(p: *mut u8) {
    unsafe { sys::det_free(p.cast()) }
}

/// `len` zeroed elements of device memory owned by the returned Buf (det_free on drop).
fn device<T: Copy>(len: usize) -> Buf<T> {
    // det_malloc gives every request, even an empty one, a block of its own
    let p = unsafe { sys::det_malloc(len * size_of::<T>()) };
    if p.is_null() {
        panic!("det_malloc: {} bytes not available", len * size_of::<T>());
    }
    unsafe { Buf::from_device(p.cast::<T>(), len, free_device) }
}

/// Host -> device copy, queued on det's stream.
unsafe fn to_device(dst: *mut u8, src: *const u8, bytes: usize) {
    unsafe { sys::det_memcpy(dst.cast(), src.cast(), bytes, STREAM) }
}

/// Device -> host copy; returns once the bytes are on the host.
unsafe fn to_host(dst: *mut u8, src: *const u8, bytes: usize) {
    unsafe {
        sys::det_memcpy(dst.cast(), src.cast(), bytes, STREAM);
        sys::det_sync();
    }
}

/// The shared device workspace: `[RESULT_BYTES][scratch]`.
struct Workspace {
    mem: Cell<Option<Buf<u8>>>,
}

impl Workspace {
    /// The base of a workspace holding at least `scratch` bytes after the result area.
    fn base(&self, scratch: usize) -> *mut u8 {
        let need = RESULT_BYTES + scratch;
        let cur = self.mem.take();
        let buf = match cur {
            Some(b) if b.len() >= need => b,
            old => {
                drop(old); // det_free waits for the ops still using it
                device::<u8>(need.next_power_of_two())
            }
        };
        let p = buf.as_mut_ptr();
        self.mem.set(Some(buf));
        p
    }
    fn scratch(&self, bytes: usize) -> *mut c_void {
        unsafe { self.base(bytes).add(RESULT_BYTES).cast() }
    }
    fn result(&self) -> *mut u8 {
        self.base(0)
    }
}

pub struct Hip {
    ws: Workspace,
}

/// A linear in the library's layout (det_linear_sizes / det_linear_repack), with the widths of its fused parts.
pub struct HipLinear {
    planes: (Buf<u8>, Buf<f32>, Buf<u16>),
    shape: (usize, usize, u32), // (N, K, bits)
    widths: Vec<usize>,
}

impl HipLinear {
    fn desc(&self) -> sys::QLinear {
        let (wq, c, m) = &self.planes;
        let (n, k, bits) = self.shape;
        sys::QLinear { wq: wq.as_ptr(), c: c.as_ptr(), m: m.as_ptr(), n: ci(n), k: ci(k), bits: bits as c_int }
    }
}

/// Where a GEMM writes, in the form det_gemm_ex takes: `y` + accumulate flag, or up to four part buffers that
/// start at the column offsets of the linear's fused widths.
struct Target {
    y: *mut f32,
    accumulate: c_int,
    nparts: c_int,
    offs: [c_int; 4],
    dsts: [*mut f32; 4],
}

impl Target {
    fn new(out: GemmOut, widths: &[usize]) -> Target {
        let mut t = Target { y: null_mut(), accumulate: 0, nparts: 0, offs: [0; 4], dsts: [null_mut(); 4] };
        match out {
            GemmOut::Write(y) => t.y = y.as_mut_ptr(),
            GemmOut::Accumulate(y) => {
                t.y = y.as_mut_ptr();
                t.accumulate = 1;
            }
            GemmOut::Parts(parts) => {
                assert!(parts.len() == widths.len() && parts.len() <= 4, "one destination per fused part, at most 4");
                let mut col = 0;
                for (i, (d, w)) in parts.iter().zip(widths).enumerate() {
                    t.offs[i] = ci(col);
                    t.dsts[i] = d.as_mut_ptr();
                    col += w;
                }
                t.nparts = ci(parts.len());
            }
        }
        t
    }
}

impl Hip {
    pub fn new() -> Self {
        let rc = unsafe { sys::det_init() };
        assert!(rc == 0, "det_init failed ({rc})");
        Hip { ws: Workspace { mem: Cell::new(None) } }
    }

    /// Bytes of device memory held through det_malloc (weights, activations, caches, the workspace).
    pub fn allocated_bytes() -> usize {
        unsafe { sys::det_allocated_bytes() }
    }
}

impl Default for Hip {
    fn default() -> Self {
        Hip::new()
    }
}

impl crate::hooks::Reader for Hip {
    unsafe fn read_bytes(&self, src: *const u8, bytes: usize, out: &mut [u8]) {
        assert!(out.len() >= bytes);
        unsafe { to_host(out.as_mut_ptr(), src, bytes) }
    }
}

impl Backend for Hip {
    type Linear = HipLinear;

    fn name(&self) -> String {
        let s = unsafe { CStr::from_ptr(sys::det_device_name()) };
        format!("hip: {}", s.to_string_lossy())
    }

    fn alloc<T: Copy>(&self, len: usize) -> Buf<T> {
        device(len)
    }

    fn write<T: Copy>(&self, b: &Buf<T>, offset: usize, data: &[T]) {
        assert!(offset <= b.len() && data.len() <= b.len() - offset, "write past the end of the buffer");
        unsafe { to_device(b.ptr_at(offset).cast(), data.as_ptr().cast(), size_of::<T>() * data.len()) }
    }

    fn read<T: Copy>(&self, b: &Buf<T>, offset: usize, out: &mut [T]) {
        assert!(offset <= b.len() && out.len() <= b.len() - offset, "read past the end of the buffer");
        unsafe { to_host(out.as_mut_ptr().cast(), b.ptr_at(offset).cast(), size_of::<T>() * out.len()) }
    }

    fn zero<T: Copy>(&self, b: &Buf<T>) {
        unsafe { sys::det_memset(b.as_mut_ptr().cast(), 0, b.bytes(), STREAM) }
    }

    fn sync(&self) {
        unsafe { sys::det_sync() }
    }

    fn linear(&self, g: &Arc<Gguf>, parts: &[&TensorInfo]) -> HipLinear {
        // the parts' det rows, concatenated along N, exactly as stored (spec/tensor.rs:49-70)
        let rows = crate::cpu::linear_parts(g, parts);
        let (k, bits) = (rows.k, rows.bits);
        let n: usize = rows.widths.iter().sum();
        let row_bytes = crate::spec::det_row_bytes(bits, k);
        // one host image of the rows, one copy to the device (a copy per row would cost a round trip per row)
        let mut image = Vec::with_capacity(n * row_bytes);
        for r in 0..n {
            image.extend_from_slice(&rows.row(r)[..row_bytes]);
        }
        let staging = device::<u8>(image.len());
        unsafe { to_device(staging.as_mut_ptr(), image.as_ptr(), image.len()) };
        drop(image);
        let (mut wq_bytes, mut c_bytes, mut m_bytes) = (0usize, 0usize, 0usize);
        unsafe { sys::hip::det_linear_sizes(ci(n), ci(k), bits as c_int, &mut wq_bytes, &mut c_bytes, &mut m_bytes) };
        let planes = (device::<u8>(wq_bytes), device::<f32>(c_bytes / 4), device::<u16>(m_bytes / 2));
        unsafe {
            sys::hip::det_linear_repack(staging.as_ptr(), ci(n), ci(k), bits as c_int, planes.0.as_mut_ptr(),
                                        planes.1.as_mut_ptr(), planes.2.as_mut_ptr(), STREAM);
        }
        drop(staging); // det_free waits for the repack to finish reading it
        HipLinear { planes, shape: (n, k, bits), widths: rows.widths.clone() }
    }

    fn linear_widths(lin: &HipLinear) -> &[usize] {
        &lin.widths
    }

    fn rmsnorm_quant(&self, x: &Buf<f32>, w: &Buf<f32>, eps: f32, m: usize, n: usize, xq: &Buf<i8>, sx: &Buf<f32>,
                     mx: &Buf<u16>) {
        // the normalised row itself is not kept (null y)
        unsafe {
            sys::det_rmsnorm_quant(x.as_ptr(), w.as_ptr(), eps, ci(m), ci(n), null_mut(), xq.as_mut_ptr(),
                                   sx.as_mut_ptr(), mx.as_mut_ptr(), STREAM)
        }
    }

    fn quant(&self, x: &Buf<f32>, m: usize, n: usize, xq: &Buf<i8>, sx: &Buf<f32>, mx: &Buf<u16>) {
        unsafe { sys::det_quant(x.as_ptr(), ci(m), ci(n), xq.as_mut_ptr(), sx.as_mut_ptr(), mx.as_mut_ptr(), STREAM) }
    }

    fn gemm(&self, lin: &HipLinear, xq: &Buf<i8>, sx: &Buf<f32>, mx: &Buf<u16>, m: usize, out: GemmOut) {
        let t = Target::new(out, &lin.widths);
        let desc = lin.desc();
        let (offs, dsts) = if t.nparts > 1 { (t.offs.as_ptr(), t.dsts.as_ptr()) } else { (null(), null()) };
        let y = if t.nparts == 1 { t.dsts[0] } else { t.y }; // one part is a plain write into it
        unsafe {
            sys::det_gemm_ex(&desc, xq.as_ptr(), sx.as_ptr(), mx.as_ptr(), ci(m), y, t.accumulate,
                             if t.nparts > 1 { t.nparts } else { 0 }, offs, dsts, STREAM)
        }
    }

    fn silu_mul_quant(&self, g: &Buf<f32>, u: &Buf<f32>, m: usize, n: usize, hq: &Buf<i8>, sh: &Buf<f32>,
                      mh: &Buf<u16>) {
        unsafe {
            sys::det_silu_mul_quant(g.as_ptr(), u.as_ptr(), ci(m), ci(n), null_mut(), hq.as_mut_ptr(),
                                    sh.as_mut_ptr(), mh.as_mut_ptr(), STREAM)
        }
    }

    fn attention(&self, l: &AttnLayer, kv: &KvCache, s: &Shape, qg: &Buf<f32>, k: &Buf<f32>, v: &Buf<f32>,
                 o: &Buf<f32>) {
        // this backend keeps no split V planes (V_PLANES is false): vlo / vhi stay null
        let cache = sys::KvCache { kq: kv.kq.as_mut_ptr(), sk: kv.sk.as_mut_ptr(), vq: kv.vq.as_mut_ptr(),
                                   capacity: ci(kv.capacity), vlo: null_mut(), vhi: null_mut() };
        let norms = sys::AttnLayer { q_norm: l.q_norm.as_ptr(), k_norm: l.k_norm.as_ptr(),
                                     v_scale: l.v_scale.as_ptr(), v_inv_scale: l.v_inv_scale.as_ptr() };
        let need = unsafe { sys::det_attn_scratch_bytes(ci(s.m), ci(s.n_h), ci(s.hd)) };
        let scratch = self.ws.scratch(need);
        unsafe {
            sys::det_attention(&norms, &cache, qg.as_ptr(), k.as_ptr(), v.as_ptr(), l.rope_cos.as_ptr(),
                               l.rope_sin.as_ptr(), ci(s.rot), s.eps, ci(s.m), ci(s.pos0), ci(s.n_h), ci(s.n_kv),
                               ci(s.hd), o.as_mut_ptr(), scratch, STREAM)
        }
    }

    fn gdn(&self, l: &GdnLayer, st: &GdnState, s: &GdnShape, qkv: &Buf<f32>, z: &Buf<f32>, a: &Buf<f32>,
           b: &Buf<f32>, on: &Buf<f32>, ex: GdnExport) {
        // gate export feeds det calibrate, which this backend does not serve
        if ex.gin.is_some() || ex.gout.is_some() {
            unimplemented!("GDN gate export (det calibrate) on the hip backend");
        }
        let params = sys::GdnLayer { conv: l.conv.as_ptr(), a: l.a.as_ptr(), dt_bias: l.dt_bias.as_ptr(),
                                     norm: l.norm.as_ptr() };
        let mut state = sys::GdnState { conv_state: st.conv_state.as_mut_ptr(), s: st.s.as_mut_ptr() };
        let (m, nk, nv, dk, dv) = (ci(s.m), ci(s.n_k), ci(s.n_v), ci(s.dk), ci(s.dv));
        let scratch = self.ws.scratch(unsafe { sys::det_gdn_scratch_bytes(m, nk, nv, dk, dv) });
        unsafe {
            sys::det_gdn(&params, &mut state, qkv.as_ptr(), z.as_ptr(), a.as_ptr(), b.as_ptr(), s.eps, m, nk, nv, dk,
                         dv, on.as_mut_ptr(), scratch, STREAM)
        }
    }

    fn argmax(&self, logits: &Buf<f32>, v: usize) -> i32 {
        let slot = self.ws.result();
        let mut idx: c_int = -1;
        unsafe {
            sys::det_argmax(logits.as_ptr(), 1, ci(v), slot.cast(), STREAM);
            to_host((&mut idx as *mut c_int).cast(), slot, size_of::<c_int>());
        }
        idx
    }

    fn sample(&self, logits: &Buf<f32>, v: usize, inv_temp: f32, top_k: usize, top_p: f32, z: u64) -> i32 {
        let mut host = vec![0f32; v];
        self.read(logits, 0, &mut host);
        crate::cpu::Cpu.sample(&Buf::host_from(&host), v, inv_temp, top_k, top_p, z)
    }
}

/// det_test_prim on this backend: `op` numbered as in det_hip.h, `m` rows of `n` (treesum writes one value per
/// row; the elementwise ops one per input).
pub fn test_prim(op: i32, x: &[f32], m: usize, n: usize) -> Vec<f32> {
    let hip = Hip::new();
    let input = hip.upload(x);
    let out = device::<f32>(x.len().max(m));
    unsafe { sys::det_test_prim(op, input.as_ptr(), ci(m), ci(n), out.as_mut_ptr(), STREAM) };
    hip.download(&out)
}
