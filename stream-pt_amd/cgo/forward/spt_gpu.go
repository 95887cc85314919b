// Package forward, GPU build: the quantized MoE path of Stream-PT's forward
// package served by libspt_moe.so (MI355X / gfx950) over cgo.
//
// This file is meant to sit in the reference's forward/ directory.  With
// the build tag spt_gpu it replaces the bodies of forwardMoE (moe.go:28),
// forwardMoEBatch (moe_batch.go:78), MulQ40Into / MulQ40BatchInto
// (q40.go:35,46) and MulQ80Argmax / MulQ80Into (q80.go:22,108); the
// reference's own definitions of those six functions move to files tagged
// !spt_gpu, so the CPU build stays the default.  When the tag is set and
// the library cannot be loaded the program fails: there is no CPU fallback.
//
// NOT COMPILED HERE: the environment this library was built in has no Go
// toolchain.  The C side it calls (include/spt_moe.h) is exercised through
// the same entry points by the Python tests.
//
//go:build spt_gpu

package forward

/*
#cgo CFLAGS: -I${SRCDIR}/../third_party/spt/include
#cgo LDFLAGS: -L${SRCDIR}/../third_party/spt/lib -lspt_moe -Wl,-rpath,${SRCDIR}/../third_party/spt/lib
#include <stdlib.h>
#include "spt_moe.h"
*/
import "C"

import (
	"context"
	"errors"
	"fmt"
	"os"
	"strconv"
	"sync"
	"sync/atomic"
	"unsafe"

	"Stream-PT/ggufindex"
	ggufmmap "Stream-PT/ggufmap"
)

// sptDevice is one context on one GPU.  Like an Engine it is not safe for
// concurrent calls (prefill.go:15): the callers below serialise on mu.
type sptDevice struct {
	mu      sync.Mutex
	ctx     *C.struct_spt_ctx
	cancel  *C.int32_t               // C memory, polled before each launch
	tensors map[string]C.spt_tensor // HBM-resident tensors by GGUF name
	xdev    unsafe.Pointer           // device staging of forwardMoE (one token)
	ydev    unsafe.Pointer
	xbytes  int
}

var (
	sptOnce   sync.Once
	sptActive *sptDevice
	sptOpenErr error
)

// activeSPT opens the device named by SPT_DEVICE (default 0) once.
func activeSPT() (*sptDevice, error) {
	sptOnce.Do(func() {
		device := 0
		if v := os.Getenv("SPT_DEVICE"); v != "" {
			n, err := strconv.Atoi(v)
			if err != nil {
				sptOpenErr = fmt.Errorf("SPT_DEVICE: %w", err)
				return
			}
			device = n
		}
		d := &sptDevice{tensors: map[string]C.spt_tensor{}}
		if rc := C.spt_ctx_create(C.int(device), nil, &d.ctx); rc != C.SPT_OK {
			sptOpenErr = sptErr(rc)
			return
		}
		d.cancel = (*C.int32_t)(C.calloc(1, 4))
		C.spt_ctx_set_cancel_flag(d.ctx, d.cancel)
		sptActive = d
	})
	return sptActive, sptOpenErr
}

func sptErr(rc C.int) error {
	if rc == C.SPT_ERR_CANCELED {
		return context.Canceled
	}
	return errors.New(C.GoString(C.spt_last_error()))
}

// run calls fn with the cancellation flag tied to ctx: set when ctx ends,
// cleared afterwards.  A canceled call returns ctx's error, as the
// reference's ctx.Err() checks do.
func (d *sptDevice) run(ctx context.Context, fn func() C.int) error {
	atomic.StoreInt32((*int32)(unsafe.Pointer(d.cancel)), 0)
	stop := context.AfterFunc(ctx, func() { atomic.StoreInt32((*int32)(unsafe.Pointer(d.cancel)), 1) })
	rc := fn()
	stop()
	atomic.StoreInt32((*int32)(unsafe.Pointer(d.cancel)), 0)
	if rc == C.SPT_ERR_CANCELED && ctx.Err() != nil {
		return ctx.Err()
	}
	if rc != C.SPT_OK {
		return sptErr(rc)
	}
	return nil
}

// PreloadSPT makes every layer's tensors and the output head resident in
// HBM at engine start: each ggufindex.Tensor's Range, as ggufindex.Open
// recorded it (ggufindex/index.go:15-26), is copied from its file unchanged
// by spt_upload_range, in place of the per-call streaming of
// WithTensorChunks / WithExpertRanges (mmap_linux.go:239,391).  The model
// is the one the engine already opened; no file is parsed again.
func PreloadSPT(model *ggufindex.Model) error {
	d, err := activeSPT()
	if err != nil {
		return err
	}
	d.mu.Lock()
	defer d.mu.Unlock()
	upload := func(t ggufindex.Tensor) error {
		if t.Name == "" {
			return nil
		}
		if _, ok := d.tensors[t.Name]; ok {
			return nil
		}
		var ct C.spt_tensor
		if len(t.Shape) > len(ct.shape) {
			return fmt.Errorf("%q: %d dimensions (at most %d are supported)", t.Name, len(t.Shape), len(ct.shape))
		}
		ct.name = C.CString(t.Name) // lives as long as the device
		ct._type = C.uint32_t(t.Type)
		ct.n_dims = C.uint32_t(len(t.Shape))
		for i, s := range t.Shape {
			ct.shape[i] = C.uint64_t(s)
		}
		path := C.CString(t.Range.File)
		defer C.free(unsafe.Pointer(path))
		if rc := C.spt_upload_range(d.ctx, path, C.uint64_t(t.Range.Start), C.uint64_t(t.Range.End), &ct); rc != C.SPT_OK {
			C.free(unsafe.Pointer(ct.name))
			return sptErr(rc)
		}
		d.tensors[t.Name] = ct
		return nil
	}
	for _, layer := range model.Layers {
		for _, t := range layer.Tensors {
			if err := upload(t); err != nil {
				return err
			}
		}
	}
	if head, ok := model.TensorByName("output.weight"); ok {
		return upload(head)
	}
	return nil
}

// tensor returns the resident copy of t, uploading it through reader on
// first use when it was not preloaded.  An unnamed tensor (an absent bias)
// is the zero descriptor, as the reference's ggufindex.Tensor{} is.
func (d *sptDevice) tensor(reader *ggufmmap.Reader, t ggufindex.Tensor) (C.spt_tensor, error) {
	if t.Name == "" {
		return C.spt_tensor{}, nil
	}
	if ct, ok := d.tensors[t.Name]; ok {
		return ct, nil
	}
	var ct C.spt_tensor
	ct.name = C.CString(t.Name) // lives as long as the device
	ct._type = C.uint32_t(t.Type)
	if len(t.Shape) > len(ct.shape) {
		return ct, fmt.Errorf("%q: %d dimensions (at most %d are supported)", t.Name, len(t.Shape), len(ct.shape))
	}
	ct.n_dims = C.uint32_t(len(t.Shape))
	for i, s := range t.Shape {
		ct.shape[i] = C.uint64_t(s)
	}
	ct.nbytes = C.uint64_t(t.Range.End - t.Range.Start)
	err := reader.WithTensor(t, func(data []byte) error {
		if len(data) == 0 {
			return nil
		}
		// data is valid only inside the callback; the upload copies it
		if rc := C.spt_tensor_upload(d.ctx, &ct, unsafe.Pointer(&data[0])); rc != C.SPT_OK {
			return sptErr(rc)
		}
		return nil
	})
	if err != nil {
		return ct, err
	}
	d.tensors[t.Name] = ct
	return ct, nil
}

func (d *sptDevice) moeLayer(reader *ggufmmap.Reader, lw *LayerWeights) (C.spt_moe_layer, error) {
	var cl C.spt_moe_layer
	for _, p := range []struct {
		dst *C.spt_tensor
		src ggufindex.Tensor
	}{
		{&cl.ffn_gate_inp, lw.FFNGateInp}, {&cl.ffn_gate_inp_bias, lw.FFNGateInpBias},
		{&cl.ffn_gate_exps, lw.FFNGateExps}, {&cl.ffn_gate_exps_bias, lw.FFNGateExpsBias},
		{&cl.ffn_up_exps, lw.FFNUpExps}, {&cl.ffn_up_exps_bias, lw.FFNUpExpsBias},
		{&cl.ffn_down_exps, lw.FFNDownExps}, {&cl.ffn_down_exps_bias, lw.FFNDownExpsBias},
	} {
		t, err := d.tensor(reader, p.src)
		if err != nil {
			return cl, err
		}
		*p.dst = t
	}
	return cl, nil
}

func moeConfig(cfg *Config) C.spt_moe_config {
	return C.spt_moe_config{
		hidden_dim: C.int32_t(cfg.HiddenDim), expert_hidden_dim: C.int32_t(cfg.ExpertHiddenDim),
		num_experts: C.int32_t(cfg.NumExperts), num_experts_used: C.int32_t(cfg.NumExpertsUsed),
	}
}

func floatPtr(v []float32) *C.float {
	if len(v) == 0 {
		return nil
	}
	return (*C.float)(unsafe.Pointer(&v[0]))
}

// forwardMoEBatch (moe_batch.go:78): same signature; the library validates
// with the reference's rules and messages, then runs route, selection,
// gate/up, SwiGLU, down and combine on the device (x and out copied through
// the context's pinned staging).  options and scratch are accepted and not
// needed: the weights are resident and the device holds the scratch.
func forwardMoEBatch(ctx context.Context, reader *ggufmmap.Reader, x []float32, cfg *Config,
	lw *LayerWeights, out []float32, batch int, options Q40Options, scratch *moeBatchScratch,
) error {
	if ctx == nil || reader == nil || cfg == nil || lw == nil {
		return fmt.Errorf("nil MoE context, reader, configuration or weights")
	}
	if err := ctx.Err(); err != nil {
		return err
	}
	d, err := activeSPT()
	if err != nil {
		return err
	}
	d.mu.Lock()
	defer d.mu.Unlock()
	cl, err := d.moeLayer(reader, lw)
	if err != nil {
		return err
	}
	cc := moeConfig(cfg)
	return d.run(ctx, func() C.int {
		return C.spt_forward_moe_batch_host(d.ctx, &cc, &cl, floatPtr(x), C.int64_t(len(x)),
			floatPtr(out), C.int64_t(len(out)), C.int64_t(batch))
	})
}

// forwardMoE (moe.go:28): one token through spt_forward_moe, which applies
// the reference's rule that an unnamed expert bias is absent (moe.go:57-62).
func forwardMoE(ctx context.Context, reader *ggufmmap.Reader, x []float32, cfg *Config,
	gateInpWeight, gateInpBias ggufindex.Tensor,
	gateExpsWeight, gateExpsBias ggufindex.Tensor,
	upExpsWeight, upExpsBias ggufindex.Tensor,
	downExpsWeight, downExpsBias ggufindex.Tensor,
	out []float32, options Q40Options, scratch *moeScratch,
) error {
	if cfg == nil {
		return fmt.Errorf("nil MoE configuration")
	}
	if ctx == nil || reader == nil {
		return fmt.Errorf("nil MoE context, reader, configuration or weights")
	}
	if err := ctx.Err(); err != nil {
		return err
	}
	d, err := activeSPT()
	if err != nil {
		return err
	}
	d.mu.Lock()
	defer d.mu.Unlock()
	lw := LayerWeights{
		FFNGateInp: gateInpWeight, FFNGateInpBias: gateInpBias,
		FFNGateExps: gateExpsWeight, FFNGateExpsBias: gateExpsBias,
		FFNUpExps: upExpsWeight, FFNUpExpsBias: upExpsBias,
		FFNDownExps: downExpsWeight, FFNDownExpsBias: downExpsBias,
	}
	cl, err := d.moeLayer(reader, &lw)
	if err != nil {
		return err
	}
	cc := moeConfig(cfg)
	// one token's x and out in device staging, kept across calls
	n := len(x) * 4
	if n != len(out)*4 || n == 0 {
		return fmt.Errorf("invalid MoE batch dimensions")
	}
	if d.xbytes < n {
		if d.xdev != nil {
			C.spt_free(d.ctx, d.xdev)
			C.spt_free(d.ctx, d.ydev)
			d.xdev, d.ydev, d.xbytes = nil, nil, 0
		}
		if rc := C.spt_alloc(d.ctx, C.uint64_t(n), &d.xdev); rc != C.SPT_OK {
			return sptErr(rc)
		}
		if rc := C.spt_alloc(d.ctx, C.uint64_t(n), &d.ydev); rc != C.SPT_OK {
			return sptErr(rc)
		}
		d.xbytes = n
	}
	if rc := C.spt_copy_h2d(d.ctx, d.xdev, unsafe.Pointer(&x[0]), C.uint64_t(n)); rc != C.SPT_OK {
		return sptErr(rc)
	}
	if err := d.run(ctx, func() C.int {
		return C.spt_forward_moe(d.ctx, &cc, &cl, (*C.float)(d.xdev), C.int64_t(len(x)),
			(*C.float)(d.ydev), C.int64_t(len(out)))
	}); err != nil {
		return err
	}
	if rc := C.spt_copy_d2h(d.ctx, unsafe.Pointer(&out[0]), d.ydev, C.uint64_t(n)); rc != C.SPT_OK {
		return sptErr(rc)
	}
	return nil
}

// MulQ40Into (q40.go:35).
func MulQ40Into(ctx context.Context, reader *ggufmmap.Reader, tensor ggufindex.Tensor,
	x, y []float32, options Q40Options) error {
	return MulQ40BatchInto(ctx, reader, tensor, x, y, 1, options)
}

// MulQ40BatchInto (q40.go:46).  options.Workers and WindowBytes are
// accepted and not needed (resident weights, the grid in place of workers).
func MulQ40BatchInto(ctx context.Context, reader *ggufmmap.Reader, tensor ggufindex.Tensor,
	x, y []float32, batch int, options Q40Options) error {
	if ctx == nil {
		return fmt.Errorf("nil context")
	}
	if reader == nil {
		return fmt.Errorf("nil GGUF reader")
	}
	if err := ctx.Err(); err != nil {
		return err
	}
	d, err := activeSPT()
	if err != nil {
		return err
	}
	d.mu.Lock()
	defer d.mu.Unlock()
	t, err := d.tensor(reader, tensor)
	if err != nil {
		return err
	}
	return d.run(ctx, func() C.int {
		return C.spt_mul_q40_batch_into_host(d.ctx, &t, floatPtr(x), C.int64_t(len(x)), floatPtr(y),
			C.int64_t(len(y)), C.int64_t(batch))
	})
}

// MulQ80Argmax (q80.go:22): the best token of W x, lowest index on ties.
func MulQ80Argmax(ctx context.Context, reader *ggufmmap.Reader, tensor ggufindex.Tensor,
	x []float32, options Q40Options) (bestToken int, bestLogit float32, err error) {
	if ctx == nil {
		return 0, 0, fmt.Errorf("nil context")
	}
	if err := ctx.Err(); err != nil {
		return 0, 0, err
	}
	d, err := activeSPT()
	if err != nil {
		return 0, 0, err
	}
	d.mu.Lock()
	defer d.mu.Unlock()
	t, err := d.tensor(reader, tensor)
	if err != nil {
		return 0, 0, err
	}
	var tok C.int64_t
	var logit C.float
	if err := d.run(ctx, func() C.int {
		return C.spt_mul_q80_argmax_host(d.ctx, &t, floatPtr(x), C.int64_t(len(x)), &tok, &logit)
	}); err != nil {
		return 0, 0, err
	}
	return int(tok), float32(logit), nil
}

// MulQ80Into (q80.go:108): all logits.
func MulQ80Into(ctx context.Context, reader *ggufmmap.Reader, tensor ggufindex.Tensor, x, y []float32,
	options Q40Options) error {
	if ctx == nil || reader == nil {
		return fmt.Errorf("nil context or reader")
	}
	if err := ctx.Err(); err != nil {
		return err
	}
	d, err := activeSPT()
	if err != nil {
		return err
	}
	d.mu.Lock()
	defer d.mu.Unlock()
	t, err := d.tensor(reader, tensor)
	if err != nil {
		return err
	}
	return d.run(ctx, func() C.int {
		return C.spt_mul_q80_into_host(d.ctx, &t, floatPtr(x), C.int64_t(len(x)), floatPtr(y), C.int64_t(len(y)))
	})
}
