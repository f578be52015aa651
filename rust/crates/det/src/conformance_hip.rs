// GEMM edge cases for `det conformance`, added to crates/det/src/conformance.rs next to `gemm` (it uses that
// module's private Rng, Report, same, fake_gguf and upload) and called from `run` after it:
//     gemm_edges(gpu, &mut r);
// Every width through every batch-size path on activation rows that are all zero, made of denormals, scaled by
// 1e-3 or ordinary; quantized by the CPU backend (quant_act_i8g) and multiplied on both backends, bit for bit.  Then
// int64 -> fp32 rounding ties in the epilogue: one nonzero code and one nonzero activation per row, with the
// multipliers chosen so that acc = m * mx lands on 2^24 + 1 and 2^24 + 3 (round to even, down and up), of both signs
// (the second group's activations are zero, so only group 0 contributes).
// UNVERIFIED: no Rust toolchain was available where this was written; the same cases run through the C ABI in the
// repository's tests (tests/test_gemm_parity.py: test_edge_rows, test_int64_to_fp32_ties).

/// Activation rows of four classes (zero, denormal, 1e-3 scaled, ordinary), cycling by row.
fn edge_acts<B: Backend>(cpu: &B, rng: &mut Rng, m: usize, k: usize) -> (Buf<i8>, Buf<f32>, Buf<u16>) {
    let x: Buf<f32> = cpu.alloc(m * k);
    fill(&x, &mut |i| match (i / k) % 4 {
        0 => 0.0,
        1 => rng.denorm(),
        2 => rng.unit() * 1e-3,
        _ => rng.unit(),
    });
    let (xq, sx, mx): (Buf<i8>, Buf<f32>, Buf<u16>) = (cpu.alloc(m * k), cpu.alloc(m), cpu.alloc(m * k / 128));
    cpu.quant(&x, m, k, &xq, &sx, &mx);
    (xq, sx, mx)
}

pub fn gemm_edges<B: Backend>(gpu: &B, r: &mut Report) {
    let cpu = Cpu;
    let mut rng = Rng(29);
    for ty in [GgmlType::Det8, GgmlType::Det6, GgmlType::Det4] {
        for (n, k) in [(200, 384), (640, 2560), (96, 17408)] {
            let g = fake_gguf(&mut rng, ty, n, k);
            let info = g.tensor("w").unwrap().clone();
            let (lc, lg) = (cpu.linear(&g, &[&info]), gpu.linear(&g, &[&info]));
            for m in [1usize, 4, 16, 17, 64, 65, 300] {
                let (xq, sx, mx) = edge_acts(&cpu, &mut rng, m, k);
                let yc: Buf<f32> = cpu.alloc(m * n);
                cpu.gemm(&lc, &xq, &sx, &mx, m, GemmOut::Write(&yc));
                let yg: Buf<f32> = gpu.alloc(m * n);
                gpu.gemm(&lg, &upload(gpu, &xq), &upload(gpu, &sx), &upload(gpu, &mx), m, GemmOut::Write(&yg));
                gpu.sync();
                r.add(format!("gemm edge rows {} n={n} k={k} m={m}", ty.name()), same(yc.host(), &gpu.download(&yg)));
            }
        }
    }
    // ties: W8 rows whose only nonzero code is +-1 at k = 0, c = 1, m = 24929 (even rows) or 10831 (odd rows);
    // activation rows whose only nonzero code is 1 at k = 0, sx = 1, mx = 673 (even tokens) or 1549 (odd tokens):
    // acc = 24929 * 673 = 2^24 + 1 (ties to 2^24) and 10831 * 1549 = 2^24 + 3 (ties to 2^24 + 4), of both signs
    let k = 256;
    let rb = GgmlType::Det8.row_bytes(k);
    let n = 64;
    let mut data = vec![0u8; n * rb];
    for row in 0..n {
        let d = &mut data[row * rb..(row + 1) * rb];
        d[0] = if row % 4 < 2 { 1 } else { (-1i8) as u8 };
        d[k..k + 4].copy_from_slice(&1.0f32.to_le_bytes());
        for gi in 0..k / 128 {
            let m: u16 = if row % 2 == 0 { 24929 } else { 10831 };
            d[k + 4 + 2 * gi..k + 6 + 2 * gi].copy_from_slice(&m.to_le_bytes());
        }
    }
    let g = tie_gguf(&data, n, k);
    let info = g.tensor("w").unwrap().clone();
    let (lc, lg) = (cpu.linear(&g, &[&info]), gpu.linear(&g, &[&info]));
    for m in [1usize, 16, 65] {
        let xq: Buf<i8> = cpu.alloc(m * k);
        let sx: Buf<f32> = cpu.alloc(m);
        let mx: Buf<u16> = cpu.alloc(m * k / 128);
        for t in 0..m {
            xq.host_mut()[t * k] = 1;              // group 1 stays zero
            sx.host_mut()[t] = 1.0;
            for gi in 0..k / 128 {
                mx.host_mut()[t * (k / 128) + gi] = if t % 2 == 0 { 673 } else { 1549 };
            }
        }
        let yc: Buf<f32> = cpu.alloc(m * n);
        cpu.gemm(&lc, &xq, &sx, &mx, m, GemmOut::Write(&yc));
        let yg: Buf<f32> = gpu.alloc(m * n);
        gpu.gemm(&lg, &upload(gpu, &xq), &upload(gpu, &sx), &upload(gpu, &mx), m, GemmOut::Write(&yg));
        gpu.sync();
        r.add(format!("gemm int64->fp32 ties m={m}"), same(yc.host(), &gpu.download(&yg)));
    }
}

/// A GGUF file holding the given W8 rows as tensor "w" (the shape fake_gguf writes).
fn tie_gguf(data: &[u8], n: usize, k: usize) -> Arc<Gguf> {
    let info = TensorInfo { name: "w".into(), dims: vec![k, n], type_id: GgmlType::Det8.id(), offset: 0 };
    let mut file = Vec::new();
    write_header(&mut file, &[("general.architecture".into(), Value::Str("test".into()))], std::slice::from_ref(&info), 32);
    file.extend_from_slice(data);
    let path = std::env::temp_dir().join(format!("det-conformance-ties-{}.gguf", std::process::id()));
    std::fs::write(&path, &file).unwrap();
    let g = Arc::new(Gguf::open(&path).unwrap());
    let _ = std::fs::remove_file(&path);
    g
}
