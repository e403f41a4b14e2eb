//! The reference's per-token call on a GPU: `KvPaging::step` then
//! `KvLayer::attention_paged` for positions 0..N of one sequence on Q8A pages
//! (Hq 32 / Hkv 8 / head_dim 128, a 40-token sliding window so that pages are
//! evicted and reused), checked against a host restatement: the stored codes
//! and scales bit for bit (`lns_decode.metal:547-593`: absmax / 127, round
//! half away from zero, clamp 127) and every output within 1e-5 of an f64
//! softmax over the dequantized window.  Needs an AMD GPU and liblnskv.so:
//! `cargo test -- --ignored`.

use lns_kv_hip::{kv_p_start, window_pages, DeviceBuffer, KvDtype, KvLayer, KvPaging, NO_PAGE};
use std::os::raw::c_void;
use std::ptr;

const HQ: usize = 32;
const HKV: usize = 8;
const D: usize = 128;

/// SplitMix64 -> values in [-2, 2).
struct Rng(u64);
impl Rng {
    fn next(&mut self) -> f32 {
        self.0 = self.0.wrapping_add(0x9E37_79B9_7F4A_7C15);
        let mut z = self.0;
        z = (z ^ (z >> 30)).wrapping_mul(0xBF58_476D_1CE4_E5B9);
        z = (z ^ (z >> 27)).wrapping_mul(0x94D0_49BB_1331_11EB);
        z ^= z >> 31;
        ((z >> 40) as f32 / (1u64 << 24) as f32) * 4.0 - 2.0
    }
}

/// One head's Q8A row as the reference's kernel writes it.
fn quantize(x: &[f32]) -> (Vec<i8>, f32) {
    let amax = x.iter().fold(0.0f32, |m, v| m.max(v.abs()));
    let sc = if amax == 0.0 { 1.0 } else { amax / 127.0 };
    (x.iter().map(|v| (v / sc).round().clamp(-127.0, 127.0) as i8).collect(), sc)
}

#[test]
#[ignore]
fn attention_paged_matches_host_restatement_on_q8a_pages() {
    let window = 40usize;
    let n_pos = 150usize;
    let layer = KvLayer::new(window_pages(window) as u32, HKV as u32, D as u32, KvDtype::Q8A).unwrap();
    let mut paging = KvPaging::new(0, window_pages(window), n_pos / 16 + 1).unwrap();
    let mut rng = Rng(7);
    // host copy of every position's dequantized K and V, [pos][kvh][d]
    let (mut kq, mut vq) = (vec![0f64; n_pos * HKV * D], vec![0f64; n_pos * HKV * D]);
    let mut q_dev = DeviceBuffer::<f32>::new(HQ * D).unwrap();
    let mut k_dev = DeviceBuffer::<f32>::new(HKV * D).unwrap();
    let mut v_dev = DeviceBuffer::<f32>::new(HKV * D).unwrap();
    let mut out_dev = DeviceBuffer::<f32>::new(HQ * D).unwrap();
    let (mut kc_dev, mut vc_dev) = (DeviceBuffer::<i8>::new(HKV * D).unwrap(), DeviceBuffer::<i8>::new(HKV * D).unwrap());
    let (mut ks_dev, mut vs_dev) = (DeviceBuffer::<f32>::new(HKV).unwrap(), DeviceBuffer::<f32>::new(HKV).unwrap());
    let scale = 1.0 / (D as f64).sqrt();
    for pos in 0..n_pos {
        let q: Vec<f32> = (0..HQ * D).map(|_| rng.next()).collect();
        let k: Vec<f32> = (0..HKV * D).map(|_| rng.next()).collect();
        let v: Vec<f32> = (0..HKV * D).map(|_| rng.next() * 0.5).collect();
        q_dev.copy_from(&q).unwrap();
        k_dev.copy_from(&k).unwrap();
        v_dev.copy_from(&v).unwrap();
        paging.step(pos, window, ptr::null_mut()).unwrap();
        let p_start = kv_p_start(pos, window);
        layer
            .dispatch_attention_paged(
                q_dev.as_ptr(),
                k_dev.as_ptr(),
                v_dev.as_ptr(),
                paging.table_dev(),
                out_dev.as_mut_ptr(),
                pos,
                D,
                HQ,
                HKV,
                p_start,
                ptr::null_mut(),
            )
            .unwrap();
        // the stored row: codes and scales bit-exact
        let row_table = DeviceBuffer::from_slice(paging.table.as_slice()).unwrap();
        layer
            .gather(
                row_table.as_ptr(),
                pos,
                1,
                kc_dev.as_mut_ptr() as *mut c_void,
                vc_dev.as_mut_ptr() as *mut c_void,
                ks_dev.as_mut_ptr(),
                vs_dev.as_mut_ptr(),
                ptr::null_mut(),
            )
            .unwrap();
        let (kc, vc) = (kc_dev.to_vec().unwrap(), vc_dev.to_vec().unwrap());
        let (ks, vs) = (ks_dev.to_vec().unwrap(), vs_dev.to_vec().unwrap());
        for h in 0..HKV {
            let (ck, sk) = quantize(&k[h * D..(h + 1) * D]);
            let (cv, sv) = quantize(&v[h * D..(h + 1) * D]);
            assert_eq!(&kc[h * D..(h + 1) * D], &ck[..], "K codes pos {pos} head {h}");
            assert_eq!(&vc[h * D..(h + 1) * D], &cv[..], "V codes pos {pos} head {h}");
            assert_eq!((ks[h].to_bits(), vs[h].to_bits()), (sk.to_bits(), sv.to_bits()), "scales pos {pos}");
            for i in 0..D {
                kq[(pos * HKV + h) * D + i] = ck[i] as f64 * sk as f64;
                vq[(pos * HKV + h) * D + i] = cv[i] as f64 * sv as f64;
            }
        }
        // f64 attention over [p_start, pos], GQA head hq -> kv head hq / 4
        let out = out_dev.to_vec().unwrap();
        for hq in 0..HQ {
            let h = hq / (HQ / HKV);
            let s: Vec<f64> = (p_start..=pos)
                .map(|t| (0..D).map(|i| q[hq * D + i] as f64 * kq[(t * HKV + h) * D + i]).sum::<f64>() * scale)
                .collect();
            let m = s.iter().cloned().fold(f64::MIN, f64::max);
            let w: Vec<f64> = s.iter().map(|x| (x - m).exp()).collect();
            let l: f64 = w.iter().sum();
            let r: Vec<f64> = (0..D)
                .map(|i| (p_start..=pos).zip(&w).map(|(t, wt)| wt * vq[(t * HKV + h) * D + i]).sum::<f64>() / l)
                .collect();
            let rmax = r.iter().fold(0.0f64, |a, x| a.max(x.abs())).max(1e-30);
            let err = (0..D).fold(0.0f64, |a, i| a.max((out[hq * D + i] as f64 - r[i]).abs())) / rmax;
            assert!(err < 1e-5, "pos {pos} head {hq}: row error {err}");
        }
        // pages of the window only, never more than window_pages(window)
        let live = paging.table.as_slice().iter().filter(|&&p| p != NO_PAGE).count();
        assert!(live <= window_pages(window));
    }
}
