//go:build !qmoe

// moe_hip_stub.go -- the CPU build (no `qmoe` tag): moeMLP never has a device
// copy, so moeMLP.forward keeps its Go body and decodeLayers its per-token
// loop (moeMLP does not implement batchMixer here); no projection has a device
// copy; packed experts cannot run (the Go path has no quantised routed
// experts) and are refused at load.
package model

import (
	"encoding/json"
	"errors"
	"os"
	"path/filepath"
)

type qmoeDev struct{}

type packedExperts struct{}

type linearDev struct{}

func (m *moeMLP) uploadQmoe(device int, selectScope int) error {
	return errors.New("built without the qmoe tag")
}

func (m *moeMLP) forwardQmoe(x []float32) []float32 { panic("built without the qmoe tag") }

func (m *moeMLP) setPostNormQmoe(w []float32, eps float32) error {
	return errors.New("built without the qmoe tag")
}

func (m *moeMLP) forwardResidualT(x []float32, T int) { panic("built without the qmoe tag") }

func (m *moeMLP) closeQmoe() {}

func (m *model) loadPackedExperts(dir string) error {
	raw, err := os.ReadFile(filepath.Join(dir, "quant.json"))
	if err != nil {
		return nil
	}
	var man struct {
		Experts []string `json:"experts"`
	}
	if json.Unmarshal(raw, &man) == nil && len(man.Experts) > 0 {
		return errors.New("packed experts need the qmoe build")
	}
	return nil
}

func newLinearDev(l *linear, q *quantLinear, out, in, device int) (*linearDev, error) {
	return nil, errors.New("built without the qmoe tag")
}

func (d *linearDev) matvec(x []float32, T int) []float32 { panic("built without the qmoe tag") }

func (d *linearDev) greedy(x []float32) int { panic("built without the qmoe tag") }

func (d *linearDev) close() {}
